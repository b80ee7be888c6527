"""Mamba2 stage M2 alone (mirror of reference atomic_ops/kernel_mamba2_a_decay.py).

``build_chunk_cumdecay_pallas(dt, A, chunk_size, interpret=False)`` keeps the
reference signature (kernel_mamba2_a_decay.py:71) and returns cumdecay
``[B, H, NT, C, P]`` float32: per chunk, sanitize(cumsum(sanitize(dt A, 20)),
1e4).  chunk_size is 64, 128 or 256 (the model's chunk, model.py:436).
``interpret`` is accepted and ignored (it selects the Pallas interpreter in
the reference).  Every computation runs in libatomic_hybrid.so; there is no
fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def stage_args(dt, n_state, chunk_size):
    """Mamba2Args for the stage entries (B and C only size the state)."""
    if not dt.is_cuda or dt.dtype not in _m._DT:
        raise TypeError("the Mamba2 stage kernels take bfloat16 or float32 dt / x / B / C on the device")
    b, l, h, p = dt.shape
    if l % chunk_size != 0:
        raise ValueError(f"seq_len={l} must be divisible by chunk_size={chunk_size}")
    return _lib.Mamba2Args(b, l, h, p, n_state, chunk_size, _m._DT[dt.dtype], _lib.ATOMIC_BF16, 0)


def stage_workspace(args, device):
    n = _lib.load().atomic_mamba2_stage_workspace_size(ctypes.byref(args))
    if n == 0:
        raise _lib.AtomicError("atomic_mamba2_stage_workspace_size: unsupported shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def build_chunk_cumdecay_pallas(dt, A, chunk_size, interpret=False):
    b, l, h, p = dt.shape
    if A.shape != (h,):
        raise ValueError(f"A must be (n_heads_ssm,)={h}, got {tuple(A.shape)}")
    dt = dt.contiguous()
    A = A.to(torch.float32).contiguous()
    # d_state only sizes the state arrays of the other stages; 128 passes the checks
    args = stage_args(dt, 128, chunk_size)
    cum = torch.empty(b, h, l // chunk_size, chunk_size, p, dtype=torch.float32, device=dt.device)
    rc = _lib.load().atomic_mamba2_chunk_cumdecay(ctypes.byref(args), _ptr(dt), _ptr(A), _ptr(cum),
                                                  _m._stream(dt.device))
    _lib.check(rc, "atomic_mamba2_chunk_cumdecay")
    return cum
