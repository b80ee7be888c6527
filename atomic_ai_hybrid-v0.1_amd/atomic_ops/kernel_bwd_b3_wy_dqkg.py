"""Kernel B3 (mirror of reference atomic_ops/kernel_bwd_b3_wy_dqkg.py).

``wy_dqkg_backward_pallas(q, k, b, w, v, gc, A, Akk, h_pre_all, v_new_all, do,
dv, dh_next_all, scale)`` keeps the reference signature
(kernel_bwd_b3_wy_dqkg.py:121) and returns its dict of dq, dk, db, dw, dv_raw,
dgc ([B, H, NT, 256, D]) and dAkk ([B, H, NT, 256, 256]), float32: the
gradients through w_pseudo, u, kg, qg and A = (I + Akk)^-1 with dA_total and
tmp clipped before the two products through A^T (:33-119).  q, k, b, w, v and
do are the inputs in block layout (bf16 or float32); gc, A, h_pre_all,
v_new_all, dv and dh_next_all float32.  Akk is only checked for its shape, as
the reference only reads its shape.  Every computation runs in
libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from ._bwd_stage import block_args, blocks_f32, operand, ptr
from .kernel_a_scores import BT


def wy_dqkg_backward_pallas(q, k, b, w, v, gc, A, Akk, h_pre_all, v_new_all, do, dv, dh_next_all, scale):
    if q.dim() != 5:
        raise ValueError("q must be [B, H, NT, 256, D]")
    B, H, NT, _, D = q.shape
    blk = (B, H, NT, BT, D)
    q = operand("q", q, blk)
    k, b, w, v = (operand(n, t, blk, q.dtype) for n, t in (("k", k), ("b", b), ("w", w), ("v", v)))
    do = operand("do", do, blk)
    gc, v_new_all, dv = (blocks_f32(n, t, blk) for n, t in (("gc", gc), ("v_new_all", v_new_all), ("dv", dv)))
    A = blocks_f32("A", A, (B, H, NT, BT, BT))
    if tuple(Akk.shape) != (B, H, NT, BT, BT):
        raise ValueError("Akk must be [B, H, NT, 256, 256]")
    h_pre_all, dh_next_all = (blocks_f32(n, t, (B, H, NT, D, D))
                              for n, t in (("h_pre_all", h_pre_all), ("dh_next_all", dh_next_all)))
    args = block_args(B, H, NT, D, D, q.dtype, do.dtype, scale)
    lib = _lib.load()
    dev = q.device
    ws = torch.empty(lib.atomic_gdn2_wy_dqkg_workspace_size(ctypes.byref(args)), dtype=torch.uint8, device=dev)
    out = {n: torch.empty(blk, dtype=torch.float32, device=dev) for n in ("dq", "dk", "db", "dw", "dv_raw", "dgc")}
    out["dAkk"] = torch.empty(B, H, NT, BT, BT, dtype=torch.float32, device=dev)
    rc = lib.atomic_gdn2_wy_dqkg_backward(
        ctypes.byref(args), ptr(q), ptr(k), ptr(b), ptr(w), ptr(v), ptr(gc), ptr(A), ptr(h_pre_all),
        ptr(v_new_all), ptr(do), ptr(dv), ptr(dh_next_all), ptr(out["dq"]), ptr(out["dk"]), ptr(out["db"]),
        ptr(out["dw"]), ptr(out["dv_raw"]), ptr(out["dgc"]), ptr(out["dAkk"]), ptr(ws), ws.numel(),
        _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_wy_dqkg_backward")
    return out
