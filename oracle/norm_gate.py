"""CPU oracle of the mixer blocks' output epilogue (RMSNorm + SiLU gate).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in PyTorch on the CPU, the inline epilogues of the reference model:
  * GDN2   (``model.py:612-613,650-653``):
        out_gate = clip(out_gate, -1e2, 1e2)
        out = RMSNorm(o).astype(bf16) ; out * silu(out_gate)
  * Mamba2 (``model.py:516-525``):
        y = y.astype(bf16) ; y = RMSNorm(y).astype(bf16)
        out = clip(y * silu(res), -3e2, 3e2)
with flax linen's RMSNorm (statistics in float32, ``x * (rsqrt(mean(x^2) +
eps) * scale)``).  With ``exact=True`` every bf16 cast is dropped and the
arithmetic runs in the inputs' dtype (float64 for the pinning tests); with
``exact=False`` the bf16 casts sit where the reference's dtypes put them,
and torch autograd gives the backward with the same dtype flow as JAX's VJP
(bf16 cotangents for the bf16 products and casts).  The clips use JAX's
min / max VJP, which splits ties evenly (cotangent factor 1/2 on the bound).
"""
from __future__ import annotations

import torch

GDN2, MAMBA2 = "gdn2", "mamba2"


class _Clip(torch.autograd.Function):
    """clip(x, -c, c) = min(max(x, -c), c) with the max / min VJP of JAX."""

    @staticmethod
    def forward(ctx, x, c):
        ctx.save_for_backward(x)
        ctx.c = c
        return x.clamp(-c, c)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        a = x.abs()
        f = torch.where(a < ctx.c, 1.0, torch.where(a == ctx.c, 0.5, 0.0)).to(g.dtype)
        return g * f, None


def rms_norm(x, weight, eps):
    """flax.linen.RMSNorm: statistics in float32 (or the input's wider dtype)."""
    xs = x if x.dtype == torch.float64 else x.to(torch.float32)
    ms = (xs * xs).mean(dim=-1, keepdim=True)
    mul = torch.rsqrt(ms + eps) * weight
    return xs * mul


def out_norm_gate(x, gate, weight, variant, eps=1e-6, exact=False):
    """The epilogue's output for x [rows, d] (o or y), gate [rows, d] (the
    out_gate projection, or res) and weight [d]."""
    bf = (lambda t: t) if exact else (lambda t: t.to(torch.bfloat16))
    if variant == MAMBA2:
        x = bf(x)                                   # y.astype(x_bc.dtype)  (:516)
    n = bf(rms_norm(x, weight, eps))                # RMSNorm(.).astype     (:519 / :652)
    g = bf(gate)
    if variant == GDN2:
        g = _Clip.apply(g, 1e2)                     # clip(out_gate, +-1e2) (:613)
    s = torch.nn.functional.silu(g)
    out = n * s
    if variant == MAMBA2:
        out = _Clip.apply(out, 3e2)                 # clip(., +-3e2)        (:524)
    return out


def out_norm_gate_grads(x, gate, weight, dout, variant, eps=1e-6, exact=False):
    """(dx, dgate, dweight) of ``out_norm_gate`` for the cotangent dout."""
    x = x.detach().clone().requires_grad_(True)
    gate = gate.detach().clone().requires_grad_(True)
    weight = weight.detach().clone().requires_grad_(True)
    out = out_norm_gate(x, gate, weight, variant, eps, exact)
    out.backward(dout.to(out.dtype))
    return x.grad, gate.grad, weight.grad
