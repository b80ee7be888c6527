"""Kernel B2 (mirror of reference atomic_ops/kernel_bwd_b2_dav.py).

``dav_backward_pallas(Aqk, v_new, do)`` keeps the reference signature
(kernel_bwd_b2_dav.py:32) and returns ``(dAqk, dv_new)``: per 256-row block,
dAqk = nan_to_num((do v_new^T) * causal) and dv_new = nan_to_num(Aqk^T do)
(:17-30), float32 [B, H, NT, 256, 256] and [B, H, NT, 256, V].  Aqk and v_new
are float32 blocks; do is the block layout of the upstream gradient (bf16 or
float32).  Every computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from ._bwd_stage import block_args, blocks_f32, operand, ptr
from .kernel_a_scores import BT


def dav_backward_pallas(Aqk, v_new, do):
    if v_new.dim() != 5:
        raise ValueError("v_new must be [B, H, NT, 256, V]")
    B, H, NT, _, V = v_new.shape
    Aqk = blocks_f32("Aqk", Aqk, (B, H, NT, BT, BT))
    v_new = blocks_f32("v_new", v_new, (B, H, NT, BT, V))
    do = operand("do", do, (B, H, NT, BT, V))
    args = block_args(B, H, NT, V, V, torch.float32, do.dtype, 1.0)
    dAqk = torch.empty_like(Aqk)
    dv_new = torch.empty_like(v_new)
    rc = _lib.load().atomic_gdn2_dav_backward(ctypes.byref(args), ptr(Aqk), ptr(v_new), ptr(do), ptr(dAqk),
                                              ptr(dv_new), _g._stream(v_new.device))
    _lib.check(rc, "atomic_gdn2_dav_backward")
    return dAqk, dv_new
