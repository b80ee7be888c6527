"""CPU oracle of the GDN2 block's prologue (the path's upstream caller).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``GatedDeltaNet2J.__call__`` of the reference model between the
projections and the GDN2 call (``model.py:574-619``), given the projection
outputs (bf16 ``[B, L, d]``, d = H * dh):

    q = silu(conv(q_lin) + conv_b_q) ; k, v likewise        (:575-592)
    v = clip(v, -50, 50)                                      (:593)
    q = grad_sanitizer(normalize(q)) ; k likewise             (:595-599)
    b = sigmoid(b_pre) ; w = sigmoid(w_pre)                   (:601-602)
    g = -exp(clip(a, -20, 20))[h] * softplus(f32(f_pre))     (:604-608)
    g = nan_to_num(g, nan=0, posinf=0, neginf=-20)            (:609)
    q, k, v, w, b, g = sanitize(., 1e3)                       (:615-619)

``conv`` is the causal depthwise convolution of ``short_causal_conv``
(``jax.lax.conv_general_dilated`` with padding (d_conv - 1, 0) and one group
per channel): out[t, c] = sum_j u[t - (d_conv - 1) + j, c] * conv_w[c, j],
with the float32 parameters cast to the activation dtype.  ``normalize(t) =
t * rsqrt(sum_c t^2 + eps^2)`` over each head's dh channels.  The gradient
sanitiser (``model.py:192-217``) is the identity forward and clips its
cotangent to +-1e3 (nan_to_num) backward.

With ``exact=True`` every cast to bf16 is dropped (float64 for the pinning
tests); otherwise bf16 roundings sit where the reference's dtypes put them:
each bf16 elementwise op rounds its result once, a bf16 reduction (the conv
taps, the head's sum of squares) accumulates in float32 and rounds once.
torch autograd then gives the backward with the same dtype flow as JAX's
VJP.  The clips use JAX's min / max VJP (ties split the cotangent evenly).
"""
from __future__ import annotations

import torch

from .norm_gate import _Clip


class _GradSanitizer(torch.autograd.Function):
    """make_grad_sanitizer (model.py:192-217): identity; the cotangent is
    nan_to_num(clip(g, -1e3, 1e3))."""

    @staticmethod
    def forward(ctx, x):
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        return torch.nan_to_num(g.clamp(-1e3, 1e3), nan=0.0, posinf=1e3, neginf=-1e3)


def _sanitize(t, c=1e3):
    """nan_to_num(clip(t, -c, c), nan=0, posinf=c, neginf=-c)  (:615-617)."""
    return torch.nan_to_num(_Clip.apply(t, c), nan=0.0, posinf=c, neginf=-c)


class _DepthwiseConv(torch.autograd.Function):
    """conv_general_dilated of a depthwise causal filter on operands of one
    dtype: products accumulated in float32 (float64 for float64 operands) and
    rounded once to the operand dtype, forward and in both VJPs (the VJPs of a
    convolution are convolutions themselves)."""

    @staticmethod
    def forward(ctx, u, wb):
        ctx.save_for_backward(u, wb)
        acc_t = torch.float64 if u.dtype == torch.float64 else torch.float32
        dc, L = wb.shape[1], u.shape[1]
        up = torch.nn.functional.pad(u.to(acc_t), (0, 0, dc - 1, 0))
        acc = sum(up[:, j:j + L, :] * wb[:, j].to(acc_t) for j in range(dc))
        return acc.to(u.dtype)

    @staticmethod
    def backward(ctx, g):
        u, wb = ctx.saved_tensors
        acc_t = torch.float64 if u.dtype == torch.float64 else torch.float32
        dc, L = wb.shape[1], u.shape[1]
        gp = torch.nn.functional.pad(g.to(acc_t), (0, 0, 0, dc - 1))     # cotangents of t .. t + dc - 1
        du = sum(gp[:, s:s + L, :] * wb[:, dc - 1 - s].to(acc_t) for s in range(dc))
        up = torch.nn.functional.pad(u.to(acc_t), (0, 0, dc - 1, 0))
        dw = torch.stack([(g.to(acc_t) * up[:, j:j + L, :]).sum((0, 1)) for j in range(dc)], dim=1)
        return du.to(u.dtype), dw.to(wb.dtype)


def causal_conv(u, w, bias, exact=False):
    """short_causal_conv (model.py:574-586): u [B, L, d], w [d, dc], bias [d];
    the float32 parameters are cast to the activation dtype."""
    dt = u.dtype if exact else torch.bfloat16
    wb, bb = w.to(dt), bias.to(dt)
    return _DepthwiseConv.apply(u, wb) + bb


def safe_normalize(t, heads, eps, exact=False):
    """t * rsqrt(sum(t * t, axis=-1) + eps^2) per head  (model.py:595-596)."""
    b, l, d = t.shape
    th = t.view(b, l, heads, d // heads)
    sq = th * th
    acc_t = t.dtype if exact else torch.float32
    ss = sq.to(acc_t).sum(-1, keepdim=True).to(t.dtype)
    r = torch.rsqrt(ss + eps ** 2)
    return (th * r).view(b, l, d)


def gdn2_prologue(q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param, heads,
                  eps=1e-6, exact=False):
    """(q, k, v, w, b, g), each [B, L, H, dh]: q..b in the activation dtype, g float32.
    conv_w: [3, d, dc] float32 (q, k, v); conv_b: [3, d] float32; a_param: [H] float32."""
    outs = []
    for i, u in enumerate((q_lin, k_lin, v_lin)):
        t = torch.nn.functional.silu(causal_conv(u, conv_w[i], conv_b[i], exact))
        if i == 2:
            t = _Clip.apply(t, 50.0)
        else:
            t = _GradSanitizer.apply(safe_normalize(t, heads, eps, exact))
        outs.append(t)
    q, k, v = outs
    bg = torch.sigmoid(b_pre)
    wg = torch.sigmoid(w_pre)
    b_, l, d = f_pre.shape
    ff = f_pre.to(torch.float64 if exact else torch.float32).view(b_, l, heads, d // heads)
    a = _Clip.apply(a_param.to(ff.dtype), 20.0)
    # jax.nn.softplus(x) = logaddexp(x, 0)
    g = -torch.exp(a)[None, None, :, None] * torch.logaddexp(ff, torch.zeros_like(ff))
    g = torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=-20.0).view(b_, l, d)
    q, k, v, wg, bg, g = (_sanitize(t) for t in (q, k, v, wg, bg, g))
    shp = (b_, l, heads, d // heads)
    return tuple(t.reshape(shp) for t in (q, k, v, wg, bg, g))


def gdn2_prologue_grads(inputs, cotangents, heads, eps=1e-6, exact=False):
    """Gradients of ``gdn2_prologue`` w.r.t. (q_lin, k_lin, v_lin, conv_w,
    conv_b, b_pre, w_pre, f_pre, a_param) for cotangents (dq, dk, dv, dw, db, dg)."""
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    outs = gdn2_prologue(*leaves, heads, eps=eps, exact=exact)
    torch.autograd.backward(outs, [c.to(o.dtype) for c, o in zip(cotangents, outs)])
    return tuple(t.grad for t in leaves)


class _ClipRange(torch.autograd.Function):
    """clip(x, lo, hi) = min(max(x, lo), hi) with JAX's max / min VJP."""

    @staticmethod
    def forward(ctx, x, lo, hi):
        ctx.save_for_backward(x)
        ctx.lo, ctx.hi = lo, hi
        return x.clamp(lo, hi)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        a = torch.where(x > ctx.lo, 1.0, torch.where(x == ctx.lo, 0.5, 0.0))
        b = torch.where(x < ctx.hi, 1.0, torch.where(x == ctx.hi, 0.5, 0.0))
        return g * (a * b).to(g.dtype), None, None


def mamba2_prologue(x_bc, conv_w, conv_b, dt_pre, b_pre, c_pre, a_log, heads, exact=False):
    """The Mamba2 block's element-wise prologue (model.py:405-433) after the
    in_proj / B_proj / C_proj / dt_proj GEMMs: (x, dt, B, C, A) with x, dt as
    [B, L, H, P] in the activation dtype, B, C [B, L, N], A float32 [H].
    conv_w: [d_inner, dc] float32; conv_b: [d_inner] float32; a_log: [H] float32."""
    x = torch.nn.functional.silu(causal_conv(x_bc, conv_w, conv_b, exact))      # :409-417
    a = _Clip.apply(a_log.to(torch.float64 if exact else torch.float32), 20.0)
    A = -torch.exp(a)                                                            # :420-422
    dt = torch.logaddexp(dt_pre, torch.zeros_like(dt_pre))                       # softplus (:425)
    lo = 1e-2 if exact else float(torch.tensor(1e-2, dtype=torch.bfloat16))    # jnp.array(1e-2, bf16)
    dt = _ClipRange.apply(dt, lo, 1.0)                                           # (:426)
    dt, B, C, x = (_sanitize(t) for t in (dt, b_pre, c_pre, x))                  # (:428-432)
    b_, l, d = x.shape
    shp = (b_, l, heads, d // heads)
    return x.reshape(shp), dt.reshape(shp), B, C, A


def mamba2_prologue_grads(inputs, cotangents, heads, exact=False):
    """Gradients of ``mamba2_prologue`` w.r.t. (x_bc, conv_w, conv_b, dt_pre,
    b_pre, c_pre, a_log) for cotangents (dx, ddt, dB, dC, dA)."""
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    outs = mamba2_prologue(*leaves, heads, exact=exact)
    torch.autograd.backward(outs, [c.to(o.dtype) for c, o in zip(cotangents, outs)])
    return tuple(t.grad for t in leaves)


class _DotBf16(torch.autograd.Function):
    """The product of flax ``Dense(dtype=bfloat16)`` (model.py:425-427): x @ W
    with float32 accumulation rounded once to the operand dtype (float64
    throughout in exact mode), and the same for both VJP products."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        acc = torch.float64 if x.dtype == torch.float64 else torch.float32
        return (x.to(acc) @ w.to(acc)).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        acc = torch.float64 if x.dtype == torch.float64 else torch.float32
        gx = (g.to(acc) @ w.to(acc).t()).to(x.dtype)
        gw = (x.to(acc).reshape(-1, x.shape[-1]).t() @ g.to(acc).reshape(-1, g.shape[-1])).to(w.dtype)
        return gx, gw


def dense(x, w, b=None, exact=False):
    """``nn.Dense(out, use_bias=b is not None, dtype=bfloat16)(x)``: the float32
    kernel [in, out] and bias cast to bf16 (autograd casts their cotangents
    back to float32), the product rounded once, the bias added in bf16."""
    dt = torch.float64 if exact else torch.bfloat16
    y = _DotBf16.apply(x, w.to(dt))
    if b is not None:
        y = y + b.to(dt)
    return y


def mamba2_projections(x_bc, w_dt, b_dt, w_b, w_c, exact=False):
    """dt_proj, B_proj, C_proj of Mamba2J (model.py:425-427) on x_bc, the first
    half of the in_proj output (:405-406): (dt_pre, b_pre, c_pre)."""
    return dense(x_bc, w_dt, b_dt, exact), dense(x_bc, w_b, None, exact), dense(x_bc, w_c, None, exact)


def mamba2_proj_prologue(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, exact=False):
    """Mamba2J's input preparation with its projections (model.py:405-433):
    (x, dt, B, C, A) as ``mamba2_prologue`` of the projection outputs."""
    dt_pre, b_pre, c_pre = mamba2_projections(x_bc, w_dt, b_dt, w_b, w_c, exact)
    return mamba2_prologue(x_bc, conv_w, conv_b, dt_pre, b_pre, c_pre, a_log, heads, exact)


def mamba2_proj_prologue_grads(inputs, cotangents, heads, exact=False):
    """Gradients of ``mamba2_proj_prologue`` w.r.t. (x_bc, conv_w, conv_b, w_dt,
    b_dt, w_b, w_c, a_log) for cotangents (dx, ddt, dB, dC, dA)."""
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    outs = mamba2_proj_prologue(*leaves, heads, exact=exact)
    torch.autograd.backward(outs, [c.to(o.dtype) for c, o in zip(cotangents, outs)])
    return tuple(t.grad for t in leaves)
