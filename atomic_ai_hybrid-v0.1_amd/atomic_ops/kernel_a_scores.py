"""Kernel A alone (mirror of reference atomic_ops/kernel_a_scores.py).

``build_chunk_scores_pallas(q, k, b, g, scale)`` keeps the reference
signature (kernel_a_scores.py:69) and returns ``(Aqk, Akk)``, float32
``[B, H, T / BT, BT, BT]`` with BT = 256, the reference's block
(kernel_a_scores.py:15-17): Aqk = scale * sum_d q_i k_j exp(clip(gc_i - gc_j,
+-20)) on causal pairs, Akk = sum_d b_i k_i k_j exp(clip(gc_i - gc_j, +-20))
on strictly causal pairs, nan_to_num'd, gc the cumsum of g over the block.
K = 128 as in the reference, or 64.  ``block=64`` gives the arrays of this
library's own 64-row chunk instead, in the inputs' dtype.  Every computation
runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g

BT = 256        # the reference's Pallas block
RUN_BLOCK = 64  # this library's chunk


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _rows(q, k, b, g):
    """The row inputs contiguous, checked like the whole-path entry."""
    if not q.is_cuda or q.dtype not in _g._DT:
        raise TypeError("q, k, b must be bf16 or fp32 device tensors")
    for t in (k, b):
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError("q, k, b must share shape and dtype")
    if g.shape != q.shape:
        raise ValueError("g must have q's shape")
    return [t.contiguous() for t in (q, k, b)] + [g.to(torch.float32).contiguous()]


def check_block(block):
    if block not in (BT, RUN_BLOCK):
        raise ValueError(f"block must be {BT} (the reference's) or {RUN_BLOCK}, got {block}")


def build_chunk_scores_pallas(q, k, b, g, scale, *, block=BT):
    check_block(block)
    q, k, b, g = _rows(q, k, b, g)
    B, T, H, K = q.shape
    NT = T // block
    args = _g.make_args(q, q, scale, chunk=block)
    dt = torch.float32 if block == BT else q.dtype
    Aqk = torch.empty(B, H, NT, block, block, dtype=dt, device=q.device)
    Akk = torch.empty_like(Aqk)
    rc = _lib.load().atomic_gdn2_chunk_scores(ctypes.byref(args), _p(q), _p(k), _p(b), _p(g), _p(Aqk), _p(Akk),
                                              _g._stream(q.device))
    _lib.check(rc, "atomic_gdn2_chunk_scores")
    return Aqk, Akk
