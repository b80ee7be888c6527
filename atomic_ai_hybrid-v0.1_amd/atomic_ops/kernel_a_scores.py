"""Kernel A alone (mirror of reference atomic_ops/kernel_a_scores.py).

``build_chunk_scores_pallas(q, k, b, g, scale)`` keeps the reference
signature (kernel_a_scores.py:69) and returns ``(Aqk, Akk)``, each
``[B, H, NT, BT, BT]``: Aqk = scale * sum_d q_i k_j exp(gc_i - gc_j) on
causal pairs, Akk = sum_d b_i k_i k_j exp(gc_i - gc_j) on strictly causal
pairs, nan_to_num'd.  BT is 64 here (the chunk of this library's kernels;
the reference's Pallas kernels fix 256 and assert d_head = 128, this one
takes K = 64 or 128); the arrays are in the inputs' dtype.  Every
computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g

BT = 64


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


def build_chunk_scores_pallas(q, k, b, g, scale):
    q, k, b, g = _rows(q, k, b, g)
    B, T, H, K = q.shape
    NT = T // BT
    args = _g.make_args(q, q, scale, chunk=BT)
    Aqk = torch.empty(B, H, NT, BT, BT, dtype=q.dtype, device=q.device)
    Akk = torch.empty_like(Aqk)
    rc = _lib.load().atomic_gdn2_chunk_scores(ctypes.byref(args), _p(q), _p(k), _p(b), _p(g), _p(Aqk), _p(Akk),
                                              _g._stream(q.device))
    _lib.check(rc, "atomic_gdn2_chunk_scores")
    return Aqk, Akk
