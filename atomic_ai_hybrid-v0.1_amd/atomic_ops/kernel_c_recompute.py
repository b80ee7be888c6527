"""Kernel C alone (mirror of reference atomic_ops/kernel_c_recompute.py).

``recompute_wy_pallas(q, k, v, w, b, g, A)`` keeps the reference signature
(kernel_c_recompute.py:91) and returns ``(w_pseudo, u, kg, qg, gc_last)``:
w_pseudo = A (b k e^gc), u = A (w v), kg = k e^(gc_last - gc), qg = q e^gc,
gc_last, each clipped to +-1e4 like the reference's kernel C
(kernel_c_recompute.py:74-82).  w_pseudo, kg, qg are [B, H, NT, BT, K],
u [B, H, NT, BT, V] in the inputs' dtype, gc_last [B, H, NT, K] float32;
BT is 64 here.  Every computation runs in libatomic_hybrid.so; there is no
fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT


def recompute_wy_pallas(q, k, v, w, b, g, A):
    _g._check_inputs(q, k, v, w, b, g)
    q, k, v, w, b, g = (t.contiguous() for t in (q, k, v, w, b, g))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // BT
    if A.shape != (B, H, NT, BT, BT) or A.dtype != q.dtype or not A.is_cuda:
        raise ValueError(f"A must be [B, H, NT, {BT}, {BT}] in q's dtype on the device")
    A = A.contiguous()
    args = _g.make_args(q, v, 1.0, chunk=BT)
    dt, dev = q.dtype, q.device
    wp, kg, qg = (torch.empty(B, H, NT, BT, K, dtype=dt, device=dev) for _ in range(3))
    u = torch.empty(B, H, NT, BT, V, dtype=dt, device=dev)
    gl = torch.empty(B, H, NT, K, dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.load().atomic_gdn2_recompute_wy(ctypes.byref(args), p(q), p(k), p(v), p(w), p(b), p(g), p(A),
                                              p(wp), p(u), p(kg), p(qg), p(gl), _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_recompute_wy")
    return wp, u, kg, qg, gl
