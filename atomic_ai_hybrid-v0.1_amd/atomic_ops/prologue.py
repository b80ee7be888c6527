"""PyTorch host side of the GDN2 block's fused prologue (the path's upstream
caller): projection outputs -> the chunk pipeline's q, k, v, w, b, g.  Every
computation runs in libatomic_hybrid.so; there is no fallback.

The reference has no standalone function for it: it is inline in
``GatedDeltaNet2J.__call__`` (``model.py:574-619``), between the
projections and ``gdn2_pallas_forward_trainable``.  ``forward`` / ``backward``
take the projection outputs (bf16 [B, L, d]), the conv parameters
(float32 [3, d, 4] and [3, d], rows q, k, v), the decay parameter a
(float32 [H]); ``GDN2Prologue`` is the autograd wrapper.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

DCONV = 4


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def make_args(b, l, heads, dhead, eps=1e-6):
    return _lib.PrologueArgs(b, l, heads, dhead, DCONV, eps)


def _check(lins, conv_w, conv_b, a_param, heads):
    q_lin = lins[0]
    if not q_lin.is_cuda:
        raise ValueError("prologue inputs must be HIP device tensors")
    b, l, d = q_lin.shape
    for t in lins:
        if t.shape != (b, l, d) or t.dtype != torch.bfloat16:
            raise TypeError("projection outputs must be bfloat16 [B, L, d]")
    if conv_w.shape != (3, d, DCONV) or conv_w.dtype != torch.float32:
        raise TypeError("conv_w must be float32 [3, d, 4]")
    if conv_b.shape != (3, d) or conv_b.dtype != torch.float32:
        raise TypeError("conv_b must be float32 [3, d]")
    if a_param.shape != (heads,) or a_param.dtype != torch.float32 or d % heads:
        raise TypeError("a_param must be float32 [H] with d divisible by H")
    return b, l, d


def forward(q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param, heads, eps=1e-6, *,
            timer=None):
    """``(q, k, v, w, b, g)`` in the [B, L, H, dh] layout of the chunk pipeline."""
    ins = [t.contiguous() for t in (q_lin, k_lin, v_lin, b_pre, w_pre, f_pre)]
    bb, l, d = _check(ins, conv_w, conv_b, a_param, heads)
    dh = d // heads
    lib = _lib.load()
    args = make_args(bb, l, heads, dh, eps)
    if timer is not None:
        args.profile = timer.arm()
    dev = q_lin.device
    shp = (bb, l, heads, dh)
    q, k, v, w, b = (torch.empty(shp, dtype=torch.bfloat16, device=dev) for _ in range(5))
    g = torch.empty(shp, dtype=torch.float32, device=dev)
    qi, ki, vi, bi, wi, fi = ins
    rc = lib.atomic_gdn2_prologue_fwd(ctypes.byref(args), _ptr(qi), _ptr(ki), _ptr(vi),
                                      _ptr(conv_w.contiguous()), _ptr(conv_b.contiguous()), _ptr(bi),
                                      _ptr(wi), _ptr(fi), _ptr(a_param.contiguous()), _ptr(q), _ptr(k),
                                      _ptr(v), _ptr(w), _ptr(b), _ptr(g), _stream(dev))
    _lib.check(rc, "atomic_gdn2_prologue_fwd")
    return q, k, v, w, b, g


def backward(q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param, heads, dq, dk, dv, dw,
             db, dg, eps=1e-6, *, workspace=None, timer=None):
    """``(dq_lin, dk_lin, dv_lin, dconv_w, dconv_b, db_pre, dw_pre, df_pre, da_param)``."""
    ins = [t.contiguous() for t in (q_lin, k_lin, v_lin, b_pre, w_pre, f_pre)]
    bb, l, d = _check(ins, conv_w, conv_b, a_param, heads)
    dh = d // heads
    lib = _lib.load()
    args = make_args(bb, l, heads, dh, eps)
    if timer is not None:
        args.profile = timer.arm()
    nbytes = lib.atomic_gdn2_prologue_workspace_size(ctypes.byref(args))
    if nbytes == 0:
        raise _lib.AtomicError("atomic_gdn2_prologue_workspace_size: unsupported shape")
    dev = q_lin.device
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    cots = [t.to(torch.bfloat16).contiguous() for t in (dq, dk, dv, dw, db)] + [dg.to(torch.float32).contiguous()]
    outs = [torch.empty(bb, l, d, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    dcw = torch.empty(3, d, DCONV, dtype=torch.float32, device=dev)
    dcb = torch.empty(3, d, dtype=torch.float32, device=dev)
    gouts = [torch.empty(bb, l, d, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    da = torch.empty(heads, dtype=torch.float32, device=dev)
    qi, ki, vi, bi, wi, fi = ins
    rc = lib.atomic_gdn2_prologue_bwd(
        ctypes.byref(args), _ptr(qi), _ptr(ki), _ptr(vi), _ptr(conv_w.contiguous()), _ptr(conv_b.contiguous()),
        _ptr(bi), _ptr(wi), _ptr(fi), _ptr(a_param.contiguous()), *(_ptr(c) for c in cots),
        *(_ptr(o) for o in outs), _ptr(dcw), _ptr(dcb), *(_ptr(o) for o in gouts), _ptr(da), _ptr(workspace),
        ctypes.c_size_t(workspace.numel()), _stream(dev))
    _lib.check(rc, "atomic_gdn2_prologue_bwd")
    return (*outs, dcw, dcb, *gouts, da)


class GDN2Prologue(torch.autograd.Function):
    """(q, k, v, w, b, g) = prologue(projection outputs, conv params, a) with the fused backward."""

    @staticmethod
    def forward(ctx, q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param, heads, eps=1e-6):
        ctx.save_for_backward(q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param)
        ctx.heads, ctx.eps = heads, eps
        return forward(q_lin, k_lin, v_lin, conv_w, conv_b, b_pre, w_pre, f_pre, a_param, heads, eps)

    @staticmethod
    def backward(ctx, dq, dk, dv, dw, db, dg):
        saved = ctx.saved_tensors
        zero = lambda t, dt_: torch.zeros(saved[0].shape[:2] + (ctx.heads, saved[0].shape[2] // ctx.heads),
                                          dtype=dt_, device=saved[0].device) if t is None else t
        grads = backward(*saved, ctx.heads, zero(dq, torch.bfloat16), zero(dk, torch.bfloat16),
                         zero(dv, torch.bfloat16), zero(dw, torch.bfloat16), zero(db, torch.bfloat16),
                         zero(dg, torch.float32), ctx.eps)
        return (*grads, None, None)


# ------------------------------------------------------------------ Mamba2
def mamba2_make_args(b, l, heads, headdim, dstate):
    return _lib.Mamba2PrologueArgs(b, l, heads, headdim, dstate, DCONV)


def _m2_check(x_bc, conv_w, conv_b, dt_pre, b_pre, c_pre, a_log, heads):
    if not x_bc.is_cuda:
        raise ValueError("prologue inputs must be HIP device tensors")
    b, l, d = x_bc.shape
    if x_bc.dtype != torch.bfloat16 or dt_pre.shape != x_bc.shape or dt_pre.dtype != torch.bfloat16:
        raise TypeError("x_bc and dt_pre must be bfloat16 [B, L, d_inner]")
    if b_pre.shape[:2] != (b, l) or c_pre.shape != b_pre.shape or b_pre.dtype != torch.bfloat16 \
            or c_pre.dtype != torch.bfloat16:
        raise TypeError("B / C projections must be bfloat16 [B, L, N]")
    if conv_w.shape != (d, DCONV) or conv_b.shape != (d,) or conv_w.dtype != torch.float32 \
            or conv_b.dtype != torch.float32:
        raise TypeError("conv_w / conv_b must be float32 [d_inner, 4] / [d_inner]")
    if a_log.shape != (heads,) or a_log.dtype != torch.float32 or d % heads:
        raise TypeError("A_log must be float32 [H] with d_inner divisible by H")
    return b, l, d, b_pre.shape[-1]


def mamba2_forward(x_bc, conv_w, conv_b, dt_pre, b_pre, c_pre, a_log, heads, *, timer=None):
    """``(x, dt, B, C, A)``: x, dt [B, L, H, P] bf16, B, C [B, L, N] bf16, A float32 [H]."""
    ins = [t.contiguous() for t in (x_bc, dt_pre, b_pre, c_pre)]
    b, l, d, n = _m2_check(ins[0], conv_w, conv_b, ins[1], ins[2], ins[3], a_log, heads)
    lib = _lib.load()
    args = mamba2_make_args(b, l, heads, d // heads, n)
    if timer is not None:
        args.profile = timer.arm()
    dev = x_bc.device
    shp = (b, l, heads, d // heads)
    x = torch.empty(shp, dtype=torch.bfloat16, device=dev)
    dt = torch.empty(shp, dtype=torch.bfloat16, device=dev)
    B = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    C = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    A = torch.empty(heads, dtype=torch.float32, device=dev)
    rc = lib.atomic_mamba2_prologue_fwd(ctypes.byref(args), _ptr(ins[0]), _ptr(conv_w.contiguous()),
                                        _ptr(conv_b.contiguous()), _ptr(ins[1]), _ptr(ins[2]), _ptr(ins[3]),
                                        _ptr(a_log.contiguous()), _ptr(x), _ptr(dt), _ptr(B), _ptr(C), _ptr(A),
                                        _stream(dev))
    _lib.check(rc, "atomic_mamba2_prologue_fwd")
    return x, dt, B, C, A


def mamba2_backward(x_bc, conv_w, conv_b, dt_pre, b_pre, c_pre, a_log, heads, dx, ddt, dB, dC, dA, *,
                    workspace=None, timer=None):
    """``(dx_bc, dconv_w, dconv_b, ddt_pre, db_pre, dc_pre, da_log)`` (dx_bc: the
    convolution path's part of x_bc's gradient)."""
    ins = [t.contiguous() for t in (x_bc, dt_pre, b_pre, c_pre)]
    b, l, d, n = _m2_check(ins[0], conv_w, conv_b, ins[1], ins[2], ins[3], a_log, heads)
    lib = _lib.load()
    args = mamba2_make_args(b, l, heads, d // heads, n)
    if timer is not None:
        args.profile = timer.arm()
    nbytes = lib.atomic_mamba2_prologue_workspace_size(ctypes.byref(args))
    if nbytes == 0:
        raise _lib.AtomicError("atomic_mamba2_prologue_workspace_size: unsupported shape")
    dev = x_bc.device
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    cots = [t.to(torch.bfloat16).contiguous() for t in (dx, ddt, dB, dC)] + [dA.to(torch.float32).contiguous()]
    dxb = torch.empty(b, l, d, dtype=torch.bfloat16, device=dev)
    dcw = torch.empty(d, DCONV, dtype=torch.float32, device=dev)
    dcb = torch.empty(d, dtype=torch.float32, device=dev)
    ddtp = torch.empty(b, l, d, dtype=torch.bfloat16, device=dev)
    dbp = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    dcp = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    dal = torch.empty(heads, dtype=torch.float32, device=dev)
    rc = lib.atomic_mamba2_prologue_bwd(
        ctypes.byref(args), _ptr(ins[0]), _ptr(conv_w.contiguous()), _ptr(conv_b.contiguous()), _ptr(ins[1]),
        _ptr(ins[2]), _ptr(ins[3]), _ptr(a_log.contiguous()), *(_ptr(c) for c in cots), _ptr(dxb), _ptr(dcw),
        _ptr(dcb), _ptr(ddtp), _ptr(dbp), _ptr(dcp), _ptr(dal), _ptr(workspace), ctypes.c_size_t(workspace.numel()),
        _stream(dev))
    _lib.check(rc, "atomic_mamba2_prologue_bwd")
    return dxb, dcw, dcb, ddtp, dbp, dcp, dal
