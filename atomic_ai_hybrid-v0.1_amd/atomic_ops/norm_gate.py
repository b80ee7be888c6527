"""PyTorch host side of the mixer blocks' fused output epilogue (RMSNorm +
SiLU gate), the path's downstream caller.  Every computation runs in
libatomic_hybrid.so; there is no fallback.

The reference has no standalone function for it: it is inline in the model,
  GDN2   ``model.py:612-613,650-653``:
      out = RMSNorm(o).astype(bf16) * silu(clip(out_gate, -1e2, 1e2))
  Mamba2 ``model.py:516-525``:
      out = clip(RMSNorm(y.astype(bf16)).astype(bf16) * silu(res), -3e2, 3e2)
followed by the block's out_proj.  ``gdn2_out_norm_gate`` /
``mamba2_out_norm_gate`` compute ``out`` (bf16) from the path's float32
output ([B, T, H, V] or [B, T, d]), the gate projection (bf16 [B, T, d]) and
the RMSNorm scale (float32 [d]); ``NormGate`` is the autograd wrapper.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

GDN2, MAMBA2 = _lib.NORM_GATE_GDN2, _lib.NORM_GATE_MAMBA2


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _prep(x, gate, weight):
    if not x.is_cuda:
        raise ValueError("epilogue inputs must be HIP device tensors")
    d = weight.shape[-1]
    if weight.dim() != 1 or weight.dtype != torch.float32:
        raise TypeError("weight must be float32 [d]")
    if x.dtype != torch.float32 or x.numel() % d != 0:
        raise TypeError("x must be float32 with the model dimension last ([..., d] or [B, T, H, V])")
    if gate.dtype != torch.bfloat16 or gate.numel() != x.numel():
        raise TypeError("gate must be bfloat16 with x's number of elements")
    rows = x.numel() // d
    return x.contiguous().view(rows, d), gate.contiguous().view(rows, d), weight.contiguous(), rows, d


def make_args(rows, d, variant, eps):
    return _lib.NormGateArgs(rows, d, variant, eps)


def forward(x, gate, weight, variant, eps=1e-6, *, timer=None):
    """``out`` [rows, d] bf16 (the shape of gate)."""
    shape = gate.shape
    x2, g2, w, rows, d = _prep(x, gate, weight)
    lib = _lib.load()
    args = make_args(rows, d, variant, eps)
    if timer is not None:
        args.profile = timer.arm()
    out = torch.empty(rows, d, dtype=torch.bfloat16, device=x.device)
    rc = lib.atomic_norm_gate_fwd(ctypes.byref(args), _ptr(x2), _ptr(g2), _ptr(w), _ptr(out),
                                  _stream(x.device))
    _lib.check(rc, "atomic_norm_gate_fwd")
    return out.view(shape)


def backward(x, gate, weight, dout, variant, eps=1e-6, *, workspace=None, timer=None):
    """``(dx, dgate, dweight)`` in x's, gate's and weight's shapes and dtypes."""
    x2, g2, w, rows, d = _prep(x, gate, weight)
    lib = _lib.load()
    args = make_args(rows, d, variant, eps)
    if timer is not None:
        args.profile = timer.arm()
    nbytes = lib.atomic_norm_gate_workspace_size(ctypes.byref(args))
    if nbytes == 0:
        raise _lib.AtomicError("atomic_norm_gate_workspace_size: unsupported shape")
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    do2 = dout.to(torch.bfloat16).contiguous().view(rows, d)
    dx = torch.empty(rows, d, dtype=torch.float32, device=x.device)
    dg = torch.empty(rows, d, dtype=torch.bfloat16, device=x.device)
    dw = torch.empty(d, dtype=torch.float32, device=x.device)
    rc = lib.atomic_norm_gate_bwd(ctypes.byref(args), _ptr(x2), _ptr(g2), _ptr(w), _ptr(do2), _ptr(dx),
                                  _ptr(dg), _ptr(dw), _ptr(workspace), ctypes.c_size_t(workspace.numel()),
                                  _stream(x.device))
    _lib.check(rc, "atomic_norm_gate_bwd")
    return dx.view(x.shape), dg.view(gate.shape), dw


class NormGate(torch.autograd.Function):
    """out = epilogue(x, gate, weight) with the fused backward."""

    @staticmethod
    def forward(ctx, x, gate, weight, variant, eps=1e-6):
        ctx.save_for_backward(x, gate, weight)
        ctx.variant, ctx.eps = variant, eps
        return forward(x, gate, weight, variant, eps)

    @staticmethod
    def backward(ctx, dout):
        x, gate, weight = ctx.saved_tensors
        dx, dg, dw = backward(x, gate, weight, dout, ctx.variant, ctx.eps)
        return dx, dg, dw, None, None


def gdn2_out_norm_gate(o, out_gate, weight, eps=1e-6):
    """RMSNorm(o).astype(bf16) * silu(clip(out_gate, -1e2, 1e2))  (model.py:612-613,650-653)."""
    return NormGate.apply(o, out_gate, weight, GDN2, eps)


def mamba2_out_norm_gate(y, res, weight, eps=1e-6):
    """clip(RMSNorm(y.astype(bf16)).astype(bf16) * silu(res), -3e2, 3e2)  (model.py:516-525)."""
    return NormGate.apply(y, res, weight, MAMBA2, eps)
