"""Kernel B1 (mirror of reference atomic_ops/kernel_bwd_b1_dhu.py).

``gdn2_dhu_backward(do, dv_partial, w_pseudo, qg, kg, gc_last, scale, dht=None)``
keeps the reference signature (kernel_bwd_b1_dhu.py:14) and returns
``(dh_all, dh0, dv_all)``: the reverse scan over 256-row blocks with dht
sanitised first and dv_new and the carry sanitised at every block (:16-44).
dh_all[:, :, n] is the carry after block n ([B, H, NT, K, V]), dh0 the carry
after block 0 and dv_all the per-block dv_new, all float32.  Every computation
runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from ._bwd_stage import block_args, blocks_f32, operand, ptr
from .kernel_a_scores import BT


def gdn2_dhu_backward(do, dv_partial, w_pseudo, qg, kg, gc_last, scale, dht=None):
    if qg.dim() != 5:
        raise ValueError("qg must be [B, H, NT, 256, K]")
    B, H, NT, _, K = qg.shape
    V = do.shape[-1]
    do = operand("do", do, (B, H, NT, BT, V))
    dv_partial = blocks_f32("dv_partial", dv_partial, (B, H, NT, BT, V))
    w_pseudo, qg, kg = (blocks_f32(n, t, (B, H, NT, BT, K))
                        for n, t in (("w_pseudo", w_pseudo), ("qg", qg), ("kg", kg)))
    gc_last = blocks_f32("gc_last", gc_last, (B, H, NT, K))
    if dht is not None:
        dht = blocks_f32("dht", dht, (B, H, K, V))
    args = block_args(B, H, NT, K, V, torch.float32, do.dtype, scale)
    dev = qg.device
    dh_all = torch.empty(B, H, NT, K, V, dtype=torch.float32, device=dev)
    dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    dv_all = torch.empty(B, H, NT, BT, V, dtype=torch.float32, device=dev)
    rc = _lib.load().atomic_gdn2_dhu_backward(ctypes.byref(args), ptr(do), ptr(dv_partial), ptr(w_pseudo), ptr(qg),
                                              ptr(kg), ptr(gc_last), ptr(dht), ptr(dh_all), ptr(dh0), ptr(dv_all),
                                              _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_dhu_backward")
    return dh_all, dh0, dv_all
