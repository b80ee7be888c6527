"""Kernel B5 (mirror of reference atomic_ops/kernel_bwd_b5_reverse_cumsum.py).

``reverse_cumsum_bwd(dgc, chunk_size)`` keeps the reference signature
(kernel_bwd_b5_reverse_cumsum.py:17) and returns dg = sanitize(suffix sum over
each block's rows) (:18-24), float32 with dgc's shape [..., chunk_size, D].
Every computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from ._bwd_stage import ptr


def reverse_cumsum_bwd(dgc, chunk_size):
    if not dgc.is_cuda or dgc.dtype != torch.float32 or dgc.dim() < 2:
        raise TypeError("dgc must be a float32 device tensor [..., chunk_size, D]")
    C, D = dgc.shape[-2:]
    if C != chunk_size or D not in (64, 128):
        raise ValueError(f"dgc must be [..., {chunk_size}, D] with D in (64, 128)")
    x = dgc.contiguous()
    blocks = x.numel() // (C * D)
    # one [blocks][C][D] array: batch = blocks, one head, seqlen = C
    args = _lib.Gdn2Args(blocks, C, 1, D, D, C, _lib.ATOMIC_F32, _lib.ATOMIC_F32, 1.0, 0)
    dg = torch.empty_like(x)
    rc = _lib.load().atomic_gdn2_reverse_cumsum_bwd(ctypes.byref(args), ptr(x), ptr(dg), _g._stream(x.device))
    _lib.check(rc, "atomic_gdn2_reverse_cumsum_bwd")
    return dg
