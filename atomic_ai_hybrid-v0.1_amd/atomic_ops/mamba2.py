"""PyTorch host side of the Mamba2 SSD chunk scan (device memory and streams
come from torch; every computation runs in libatomic_hybrid.so).

Layouts follow the reference (``atomic_ops/kernel_mamba2_trainable_B6.py:137``):
dt, x: [B, T, H, P]; Bm, Cm: [B, T, N] (shared by all heads); A: [H] float32;
state0 / state_final: [B, H, P, N] float32; y: [B, T, H, P] float32.
dt, x, Bm, Cm are bfloat16 or float32 (one dtype); float32 operands run the
library's float32 staged chain at the given chunk (M2 -> M3 -> M4 forward,
MB1 + MB3 -> MB4 backward), bfloat16 ones the fused whole-path kernels.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DT = {torch.float32: _lib.ATOMIC_F32, torch.bfloat16: _lib.ATOMIC_BF16}
M2_SAVE, M2_REUSE, M2_SANITIZE_STATE0 = 1, 2, 4


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _check(dt, x, Bm, Cm, A):
    if not dt.is_cuda:
        raise ValueError("Mamba2 inputs must be HIP device tensors")
    if dt.dtype not in _DT:
        raise TypeError("the Mamba2 kernels take bfloat16 or float32 dt / x / B / C")
    if x.shape != dt.shape or x.dtype != dt.dtype:
        raise ValueError("x must match dt")
    b, l, h, p = dt.shape
    if Bm.shape[:2] != (b, l) or Cm.shape != Bm.shape or Bm.dtype != dt.dtype or Cm.dtype != dt.dtype:
        raise ValueError("B and C must be [B, T, N] with dt's dtype")
    if A.shape != (h,) or A.dtype != torch.float32:
        raise ValueError("A must be float32 [H]")


def _rows_of(args, tensors):
    """_lib.row_view of dt, x, B, C (and dy), their strides into args.row_stride."""
    out = []
    for i, t in enumerate(tensors):
        t2, s = _lib.row_view(t)
        args.row_stride[i] = s
        out.append(t2)
    return out


def make_args(dt, Bm, chunk_size, *, dy_dtype=None, flags=0):
    b, l, h, p = dt.shape
    if l % chunk_size != 0:
        raise ValueError(f"seq_len={l} must be divisible by chunk_size={chunk_size}")
    return _lib.Mamba2Args(b, l, h, p, Bm.shape[-1], chunk_size, _DT[dt.dtype],
                           _DT[dy_dtype if dy_dtype is not None else dt.dtype], flags)


def workspace_bytes(args):
    n = _lib.load().atomic_mamba2_workspace_size(ctypes.byref(args))
    if n == 0:
        raise _lib.AtomicError("atomic_mamba2_workspace_size: unsupported shape")
    return n


def forward(dt, x, Bm, Cm, A, chunk_size, state0=None, *, save=False, workspace=None, timer=None,
            diag=None, sanitize_state0=False):
    """Returns ``(y, state_final, workspace)``.  ``diag`` (an
    ``_lib.StageReports`` over ``_lib.MAMBA2_DIAG_STAGES``) receives the
    forward's per-stage reports.  ``sanitize_state0`` clips state0 to +-1e4
    and nan_to_nums it first, as the reference's staged combine does
    (kernel_mamba2_c_interchunk.py:56-58)."""
    _check(dt, x, Bm, Cm, A)
    lib = _lib.load()
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    flags = (M2_SAVE if save else 0) | (M2_SANITIZE_STATE0 if sanitize_state0 else 0)
    args = make_args(dt, Bm, chunk_size, flags=flags)
    dt, x, Bm, Cm = _rows_of(args, (dt, x, Bm, Cm))
    A = A.contiguous()
    if timer is not None:
        args.profile = timer.arm()
    if diag is not None:
        args.diag = diag.ptr
    if workspace is None:
        workspace = torch.empty(workspace_bytes(args), dtype=torch.uint8, device=dt.device)
    if state0 is not None:
        state0 = state0.to(torch.float32).contiguous()
    y = torch.empty(b, l, h, p, dtype=torch.float32, device=dt.device)
    state_final = torch.empty(b, h, p, n, dtype=torch.float32, device=dt.device)
    rc = lib.atomic_mamba2_fwd(ctypes.byref(args), _ptr(dt), _ptr(x), _ptr(Bm), _ptr(Cm), _ptr(A),
                               _ptr(state0), _ptr(y), _ptr(state_final), _ptr(workspace),
                               ctypes.c_size_t(workspace.numel()), _stream(dt.device))
    _lib.check(rc, "atomic_mamba2_fwd")
    return y, state_final, workspace


def backward(dt, x, Bm, Cm, A, chunk_size, dy, dstate_final=None, state0=None, *, workspace=None,
             reuse=False, timer=None, diag=None, sanitize_state0=False):
    """Gradients ``(ddt, dx, dB, dC, dA, dstate0)`` (MB0 semantics) in the
    primals' dtypes (dA, dstate0 float32).  ``reuse`` declares that
    ``workspace`` holds the forward of the same inputs; the library checks
    that by the input addresses, so an input that has to be copied here (not
    contiguous and not row-strided, or state0 not float32) turns reuse into a
    recompute.  ``sanitize_state0`` must match the forward's."""
    _check(dt, x, Bm, Cm, A)
    lib = _lib.load()
    if dy.dtype not in _DT:
        dy = dy.to(torch.float32)
    args = make_args(dt, Bm, chunk_size, dy_dtype=dy.dtype)
    seen = (dt, x, Bm, Cm)
    dt, x, Bm, Cm, dy = _rows_of(args, seen + (dy,))
    if any(a is not b_ for a, b_ in zip((dt, x, Bm, Cm), seen)) or not A.is_contiguous() or \
            (state0 is not None and (state0.dtype != torch.float32 or not state0.is_contiguous())):
        reuse = False
    A = A.contiguous()
    args.flags = (M2_REUSE if reuse else 0) | (M2_SANITIZE_STATE0 if sanitize_state0 else 0)
    if timer is not None:
        args.profile = timer.arm()
    if diag is not None:
        args.diag = diag.ptr
    if workspace is None:
        workspace = torch.empty(workspace_bytes(args), dtype=torch.uint8, device=dt.device)
    if state0 is not None:
        state0 = state0.to(torch.float32).contiguous()
    if dstate_final is not None:
        dstate_final = dstate_final.to(torch.float32).contiguous()
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    # the gradients are dense
    ddt, dx = (torch.empty(dt.shape, dtype=dt.dtype, device=dt.device) for _ in range(2))
    dB, dC = (torch.empty(Bm.shape, dtype=Bm.dtype, device=Bm.device) for _ in range(2))
    dA = torch.empty(h, dtype=torch.float32, device=dt.device)
    dstate0 = torch.empty(b, h, p, n, dtype=torch.float32, device=dt.device)
    rc = lib.atomic_mamba2_bwd(ctypes.byref(args), _ptr(dt), _ptr(x), _ptr(Bm), _ptr(Cm), _ptr(A),
                               _ptr(state0), _ptr(dy), _ptr(dstate_final), _ptr(ddt), _ptr(dx),
                               _ptr(dB), _ptr(dC), _ptr(dA), _ptr(dstate0), _ptr(workspace),
                               ctypes.c_size_t(workspace.numel()), _stream(dt.device))
    _lib.check(rc, "atomic_mamba2_bwd")
    return ddt, dx, dB, dC, dA, dstate0
