"""Kernel C alone (mirror of reference atomic_ops/kernel_c_recompute.py).

``recompute_wy_pallas(q, k, v, w, b, g, A)`` keeps the reference signature
(kernel_c_recompute.py:91) and returns ``(w_pseudo, u, kg, qg, gc_last)``:
w_pseudo = A (b k e^gc), u = A (w v), kg = k e^(gc_last - gc), qg = q e^gc
and gc_last, each clipped to +-1e4 like the reference's kernel C
(kernel_c_recompute.py:68-82).  The block is A's: for the reference's float32
``[B, H, NT, 256, 256]`` A the results are float32 [B, H, NT, 256, K]
(u [.., V]) with w v formed in float32 as the reference does (:56-62); for
this library's 64-row A (in the inputs' dtype) they are in the inputs' dtype.
gc_last is [B, H, NT, K] float32.  Every computation runs in
libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT, RUN_BLOCK


def recompute_wy_pallas(q, k, v, w, b, g, A):
    _g._check_inputs(q, k, v, w, b, g)
    q, k, v, w, b, g = (t.contiguous() for t in (q, k, v, w, b, g))
    B, T, H, K = q.shape
    V = v.shape[-1]
    blk = A.shape[-1]
    if blk not in (BT, RUN_BLOCK) or T % blk != 0:
        raise ValueError(f"A must be [B, H, T/{BT}, {BT}, {BT}] or [B, H, T/{RUN_BLOCK}, {RUN_BLOCK}, {RUN_BLOCK}]")
    NT = T // blk
    dt = torch.float32 if blk == BT else q.dtype
    if A.shape != (B, H, NT, blk, blk) or A.dtype != dt or not A.is_cuda:
        raise ValueError(f"A must be [B, H, NT, {blk}, {blk}] in {dt} on the device")
    A = A.contiguous()
    args = _g.make_args(q, v, 1.0, chunk=blk)
    dev = q.device
    wp, kg, qg = (torch.empty(B, H, NT, blk, K, dtype=dt, device=dev) for _ in range(3))
    u = torch.empty(B, H, NT, blk, V, dtype=dt, device=dev)
    gl = torch.empty(B, H, NT, K, dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.load().atomic_gdn2_recompute_wy(ctypes.byref(args), p(q), p(k), p(v), p(w), p(b), p(g), p(A),
                                              p(wp), p(u), p(kg), p(qg), p(gl), _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_recompute_wy")
    return wp, u, kg, qg, gl
