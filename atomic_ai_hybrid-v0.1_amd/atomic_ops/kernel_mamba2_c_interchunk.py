"""Mamba2 stage M4 and the staged forward (mirror of reference
atomic_ops/kernel_mamba2_c_interchunk.py).

``mamba2_inter_chunk_combine(y_diag, state_end, cumdecay, C, chunk_size,
state0=None)`` keeps the reference signature (kernel_mamba2_c_interchunk.py:38)
and returns ``(y [B, T, H, P], state_final [B, H, P, N])`` float32: the
sequential state pass over the chunks (state0 sanitised) and y =
sanitize(y_diag + y_off).  ``mamba2_pallas_forward(dt, x, B, C, A,
chunk_size, state0=None, interpret=False)`` chains M2 -> M3 -> M4 like the
reference (:90-100).  chunk_size is 64, 128 or 256.  Every computation runs in
libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m
from .kernel_mamba2_a_decay import _ptr, build_chunk_cumdecay_pallas, stage_workspace
from .kernel_mamba2_b_intra import intra_chunk_ssd_pallas


def mamba2_inter_chunk_combine(y_diag, state_end, cumdecay, C, chunk_size, state0=None):
    b, l, h, p = y_diag.shape
    n = C.shape[-1]
    nt = l // chunk_size if l % chunk_size == 0 else -1
    if state_end.shape != (b, h, nt, p, n) or cumdecay.shape != (b, h, nt, chunk_size, p) \
            or C.shape != (b, l, n):
        raise ValueError("inconsistent stage array shapes")
    if not C.is_cuda or C.dtype not in _m._DT:
        raise TypeError("C must be a bfloat16 or float32 device tensor")
    args = _lib.Mamba2Args(b, l, h, p, n, chunk_size, _m._DT[C.dtype], _lib.ATOMIC_BF16, 0)
    y_diag, state_end, cumdecay = (t.to(torch.float32).contiguous() for t in (y_diag, state_end, cumdecay))
    C = C.contiguous()
    if state0 is not None:
        state0 = state0.to(torch.float32).contiguous()
    ws = stage_workspace(args, C.device)
    y = torch.empty(b, l, h, p, dtype=torch.float32, device=C.device)
    state_final = torch.empty(b, h, p, n, dtype=torch.float32, device=C.device)
    rc = _lib.load().atomic_mamba2_inter_chunk_combine(ctypes.byref(args), _ptr(y_diag), _ptr(state_end),
                                                       _ptr(cumdecay), _ptr(C), _ptr(state0), _ptr(y),
                                                       _ptr(state_final), _ptr(ws), ctypes.c_size_t(ws.numel()),
                                                       _m._stream(C.device))
    _lib.check(rc, "atomic_mamba2_inter_chunk_combine")
    return y, state_final


def mamba2_pallas_forward(dt, x, B, C, A, chunk_size, state0=None, interpret=False):
    cumdecay = build_chunk_cumdecay_pallas(dt, A, chunk_size)
    y_diag, state_end = intra_chunk_ssd_pallas(dt, x, B, C, cumdecay, chunk_size)
    return mamba2_inter_chunk_combine(y_diag, state_end, cumdecay, C, chunk_size, state0=state0)
