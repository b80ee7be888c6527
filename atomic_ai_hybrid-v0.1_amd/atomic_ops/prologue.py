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


# ------------------------------------------------- Mamba2 with its projections
def mamba2_proj_make_args(b, l, heads, headdim, dstate, in_stride):
    return _lib.Mamba2ProjArgs(b, l, heads, headdim, dstate, DCONV, in_stride)


def _x_bc_view(in_proj_or_x_bc, d_inner):
    """x_bc as a [B, L, d_inner] view whose rows may be strided (the first half
    of the in_proj output, model.py:405-406); returns (view, row stride)."""
    t = in_proj_or_x_bc
    if t.dim() != 3 or t.shape[-1] < d_inner or t.stride(-1) != 1 or t.stride(0) != t.shape[1] * t.stride(1):
        raise TypeError("x_bc must be [B, L, >= d_inner] with unit column stride and rows of one stride")
    return t[..., :d_inner], t.stride(1)


def _m2x_check(x_bc, ld, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads):
    if not x_bc.is_cuda:
        raise ValueError("prologue inputs must be HIP device tensors")
    if x_bc.dtype != torch.bfloat16:
        raise TypeError("x_bc must be bfloat16")
    b, l, d = x_bc.shape
    n = w_b.shape[-1]
    if w_dt.shape != (d, d) or b_dt.shape != (d,) or w_b.shape != (d, n) or w_c.shape != (d, n):
        raise TypeError("W_dt [d, d], b_dt [d], W_B / W_C [d, N] expected (the Dense [in, out] layout)")
    for t in (w_dt, b_dt, w_b, w_c, conv_w, conv_b, a_log):
        if t.dtype != torch.float32:
            raise TypeError("parameters must be float32")
    if conv_w.shape != (d, DCONV) or conv_b.shape != (d,) or a_log.shape != (heads,) or d % heads:
        raise TypeError("conv_w [d, 4], conv_b [d], A_log [H] with d divisible by H expected")
    return b, l, d, n


def mamba2_proj_forward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, *, save=False,
                        workspace=None, timer=None):
    """Mamba2J's input preparation from the in_proj output (model.py:405-433):
    ``(x, dt, B, C, A)`` -- x, dt [B, L, H, P] bf16, B, C [B, L, N] bf16, A
    float32 [H] -- and, with ``save``, the projection outputs ``(dt_pre,
    b_pre, c_pre)`` the backward takes.  ``x_bc`` may be the whole in_proj
    output [B, L, 2 d_inner] or any row-strided view whose first d_inner
    columns are x_bc; it is read in place."""
    d = w_dt.shape[0]
    xv, ld = _x_bc_view(x_bc, d)
    b, l, d, n = _m2x_check(xv, ld, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads)
    lib = _lib.load()
    args = mamba2_proj_make_args(b, l, heads, d // heads, n, ld)
    if timer is not None:
        args.profile = timer.arm()
    nbytes = lib.atomic_mamba2_proj_workspace_size(ctypes.byref(args), 0)
    if nbytes == 0:
        raise _lib.AtomicError("atomic_mamba2_proj_workspace_size: unsupported shape")
    dev = xv.device
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    shp = (b, l, heads, d // heads)
    x = torch.empty(shp, dtype=torch.bfloat16, device=dev)
    dt = torch.empty(shp, dtype=torch.bfloat16, device=dev)
    B = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    C = torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)
    A = torch.empty(heads, dtype=torch.float32, device=dev)
    pres = (torch.empty(b, l, d, dtype=torch.bfloat16, device=dev),
            torch.empty(b, l, n, dtype=torch.bfloat16, device=dev),
            torch.empty(b, l, n, dtype=torch.bfloat16, device=dev)) if save else (None, None, None)
    nul = ctypes.c_void_p(0)
    params = [t.contiguous() for t in (conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log)]
    rc = lib.atomic_mamba2_proj_fwd(ctypes.byref(args), _ptr(xv), *(_ptr(t) for t in params), _ptr(x), _ptr(dt),
                                    _ptr(B), _ptr(C), _ptr(A), *((_ptr(t) if t is not None else nul) for t in pres),
                                    _ptr(workspace), ctypes.c_size_t(workspace.numel()), _stream(dev))
    _lib.check(rc, "atomic_mamba2_proj_fwd")
    if save:
        return (x, dt, B, C, A), pres
    return x, dt, B, C, A


def mamba2_proj_backward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, pres, dx, ddt, dB, dC, dA, *,
                         dx_bc=None, workspace=None, timer=None):
    """Gradients ``(dx_bc, dconv_w, dconv_b, dw_dt, db_dt, dw_b, dw_c, da_log)``
    for the cotangents of ``mamba2_proj_forward``'s outputs; ``pres`` are its
    saved projection outputs.  dx_bc is x_bc's whole gradient; pass ``dx_bc``
    (a tensor strided like ``x_bc``, e.g. the in_proj gradient) to have its
    first d_inner columns written in place."""
    d = w_dt.shape[0]
    xv, ld = _x_bc_view(x_bc, d)
    b, l, d, n = _m2x_check(xv, ld, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads)
    lib = _lib.load()
    dev = xv.device
    if dx_bc is None:
        buf = torch.empty((b * l - 1) * ld + d, dtype=torch.bfloat16, device=dev)
        out = buf.as_strided((b, l, d), (l * ld, ld, 1))
    else:
        if dx_bc.dtype != torch.bfloat16 or dx_bc.dim() != 3 or dx_bc.shape[:2] != (b, l) \
                or dx_bc.shape[-1] < d or dx_bc.stride() != (l * ld, ld, 1):
            raise TypeError("dx_bc must be bfloat16 [B, L, >= d_inner] with the rows of x_bc")
        out = dx_bc[..., :d]
    args = mamba2_proj_make_args(b, l, heads, d // heads, n, ld)
    if timer is not None:
        args.profile = timer.arm()
    nbytes = lib.atomic_mamba2_proj_workspace_size(ctypes.byref(args), 1)
    if nbytes == 0:
        raise _lib.AtomicError("atomic_mamba2_proj_workspace_size: unsupported shape")
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    pres = [t.contiguous() for t in pres]
    cots = [t.to(torch.bfloat16).contiguous() for t in (dx, ddt, dB, dC)] + [dA.to(torch.float32).contiguous()]
    params = [t.contiguous() for t in (conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log)]
    dcw = torch.empty(d, DCONV, dtype=torch.float32, device=dev)
    dcb = torch.empty(d, dtype=torch.float32, device=dev)
    dwdt = torch.empty(d, d, dtype=torch.float32, device=dev)
    dbdt = torch.empty(d, dtype=torch.float32, device=dev)
    dwb = torch.empty(d, n, dtype=torch.float32, device=dev)
    dwc = torch.empty(d, n, dtype=torch.float32, device=dev)
    dal = torch.empty(heads, dtype=torch.float32, device=dev)
    rc = lib.atomic_mamba2_proj_bwd(
        ctypes.byref(args), _ptr(xv), *(_ptr(t) for t in params), *(_ptr(t) for t in pres),
        *(_ptr(c) for c in cots), _ptr(out), _ptr(dcw), _ptr(dcb), _ptr(dwdt), _ptr(dbdt), _ptr(dwb),
        _ptr(dwc), _ptr(dal), _ptr(workspace), ctypes.c_size_t(workspace.numel()), _stream(dev))
    _lib.check(rc, "atomic_mamba2_proj_bwd")
    return out, dcw, dcb, dwdt, dbdt, dwb, dwc, dal


class Mamba2ProjPrologue(torch.autograd.Function):
    """(x, dt, B, C, A) = Mamba2J's input preparation from x_bc (a row-strided
    view of the in_proj output) and the conv / dt_proj / B_proj / C_proj / A_log
    parameters, with the fused backward."""

    @staticmethod
    def forward(ctx, x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads):
        outs, pres = mamba2_proj_forward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, save=True)
        ctx.save_for_backward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, *pres)
        ctx.heads = heads
        return outs

    @staticmethod
    def backward(ctx, dx, ddt, dB, dC, dA):
        x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, *pres = ctx.saved_tensors
        zero = lambda g, ref, dt_: torch.zeros(ref, dtype=dt_, device=x_bc.device) if g is None else g
        d, n, heads = w_dt.shape[0], w_b.shape[1], ctx.heads
        b, l = x_bc.shape[:2]
        shp = (b, l, heads, d // heads)
        cots = (zero(dx, shp, torch.bfloat16), zero(ddt, shp, torch.bfloat16), zero(dB, (b, l, n), torch.bfloat16),
                zero(dC, (b, l, n), torch.bfloat16), zero(dA, (heads,), torch.float32))
        if x_bc.shape[-1] == d:
            g = mamba2_proj_backward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, pres, *cots)
            return (*g, None)
        # x_bc is the whole in_proj output: its other columns get a zero gradient
        full = torch.zeros(x_bc.shape, dtype=torch.bfloat16, device=x_bc.device)
        if full.stride() == x_bc.stride():
            g = mamba2_proj_backward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, pres, *cots,
                                     dx_bc=full)
        else:
            g = mamba2_proj_backward(x_bc, conv_w, conv_b, w_dt, b_dt, w_b, w_c, a_log, heads, pres, *cots)
            full[..., :d] = g[0]
        return (full, *g[1:], None)
