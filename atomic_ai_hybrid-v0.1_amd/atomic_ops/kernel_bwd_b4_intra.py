"""Kernel B4 (mirror of reference atomic_ops/kernel_bwd_b4_intra.py).

``intra_backward_pallas(dAqk, dAkk, q, k, b, g, scale)`` keeps the reference
signature (kernel_bwd_b4_intra.py:135) and returns ``(dq, dk, db, dgc)``,
float32 [B, H, NT, 256, K]: kernel A's backward over its 128-row sub-block
pairs with pairwise exp(clip(gc_i - gc_j, +-20)), the clip mask on the dgc
terms and a clip to +-1e4 after every accumulation (:57-132).  q, k, b are the
[B, T, H, K] inputs (bf16 or float32), g float32; dAqk, dAkk float32
[B, H, NT, 256, 256].  Like the reference it takes K = 128 only (:137).
Every computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from ._bwd_stage import blocks_f32, ptr
from .kernel_a_scores import BT


def intra_backward_pallas(dAqk, dAkk, q, k, b, g, scale):
    B, T, H, D = q.shape
    if D != 128:
        raise ValueError(f"Kernel B4 assumes d_head=128; got D={D}")      # kernel_bwd_b4_intra.py:137
    if T % BT != 0:
        raise ValueError(f"seq_len={T} must be divisible by BT={BT}")     # :138
    _g._check_inputs(q, k, q, q, b, g)
    NT = T // BT
    dAqk = blocks_f32("dAqk", dAqk, (B, H, NT, BT, BT))
    dAkk = blocks_f32("dAkk", dAkk, (B, H, NT, BT, BT))
    q, k, b, g = (t.contiguous() for t in (q, k, b, g))
    args = _g.make_args(q, q, scale, chunk=BT)
    dev = q.device
    dq, dk, db, dgc = (torch.empty(B, H, NT, BT, D, dtype=torch.float32, device=dev) for _ in range(4))
    rc = _lib.load().atomic_gdn2_intra_backward(ctypes.byref(args), ptr(dAqk), ptr(dAkk), ptr(q), ptr(k), ptr(b),
                                                ptr(g), ptr(dq), ptr(dk), ptr(db), ptr(dgc), _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_intra_backward")
    return dq, dk, db, dgc
