"""Mamba2 stage M3 alone (mirror of reference atomic_ops/kernel_mamba2_b_intra.py).

``intra_chunk_ssd_pallas(dt, x, B, C, cumdecay, chunk_size, interpret=False)``
keeps the reference signature (kernel_mamba2_b_intra.py:119) and returns
``(y_diag [B, T, H, P], state_end [B, H, NT, P, N])``, float32, from the
given cumdecay: y_diag_i = sum_{j<=i} exp(clip(cum_i - cum_j, +-20))
CB_ij dBx_j and state_end = B^T sanitize(dBx exp(clip(cum_last - cum,
+-20))), with the reference stage kernel's clips (no 1e6 caps).  chunk_size
is 64, 128 or 256; at 256 the sum runs over the reference's two 128-row
sub-blocks, each sub-block's part sanitised before the next is added
(kernel_mamba2_b_intra.py:61-62,86-108).  Every computation runs in libatomic_hybrid.so; there is no
fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m
from .kernel_mamba2_a_decay import _ptr, stage_args, stage_workspace


def intra_chunk_ssd_pallas(dt, x, B, C, cumdecay, chunk_size, interpret=False):
    b, l, h, p = dt.shape
    n = B.shape[-1]
    nt = l // chunk_size if l % chunk_size == 0 else -1
    if x.shape != dt.shape or x.dtype != dt.dtype or B.shape != (b, l, n) or C.shape != B.shape \
            or B.dtype != dt.dtype or C.dtype != dt.dtype:
        raise ValueError("x must match dt; B and C must be [B, T, N] in dt's dtype")
    if cumdecay.shape != (b, h, nt, chunk_size, p):
        raise ValueError(f"cumdecay must be [B, H, NT, {chunk_size}, P], got {tuple(cumdecay.shape)}")
    args = stage_args(dt, n, chunk_size)
    dt, x, B, C = (t.contiguous() for t in (dt, x, B, C))
    cum = cumdecay.to(torch.float32).contiguous()
    ws = stage_workspace(args, dt.device)
    y_diag = torch.empty(b, l, h, p, dtype=torch.float32, device=dt.device)
    state_end = torch.empty(b, h, nt, p, n, dtype=torch.float32, device=dt.device)
    rc = _lib.load().atomic_mamba2_intra_chunk_ssd(ctypes.byref(args), _ptr(dt), _ptr(x), _ptr(B), _ptr(C),
                                                   _ptr(cum), _ptr(y_diag), _ptr(state_end), _ptr(ws),
                                                   ctypes.c_size_t(ws.numel()), _m._stream(dt.device))
    _lib.check(rc, "atomic_mamba2_intra_chunk_ssd")
    return y_diag, state_end
