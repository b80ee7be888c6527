"""Stage-level GDN2 forward (mirror of reference atomic_ops/kernel_d_pipeline.py).

``gdn2_inter_chunk_combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None,
debug_tag="")`` keeps the reference signature (kernel_d_pipeline.py:94) and
returns ``(o, h_final)`` with o per chunk, ``[B, H, NT, BT, V]`` float32;
``build_chunk_wy(q, k, v, w, b, g, scale)`` runs the reference's kernels
A + B + C (build_chunk_scores_pallas, wy_solve_pallas, recompute_wy_pallas:
kernel_a_scores.py:69, kernel_b_solve.py:151, kernel_c_recompute.py:91) as one
pass and returns ``(Aqk, A, w_pseudo, u, kg, qg, gc_last)``;
``gdn2_inter_chunk_combine_with_state`` and ``gdn2_pallas_forward_with_residuals``
(kernel_d_pipeline.py:127,199) also return the scan's per-chunk states.  The
combine runs at the block of its arrays: the reference's 256 rows (float32
arrays, the kernels A, B, C mirrors' default) or this library's 64 (arrays
in the inputs' dtype, as ``build_chunk_wy`` returns them; gc_last float32).
Every computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT as REF_BLOCK, check_block
from .kernel_trainable_B6 import gdn2_pallas_forward  # noqa: F401  (the whole staged forward)

BT = 64   # the block of build_chunk_wy


def build_chunk_wy(q, k, v, w, b, g, scale):
    """Per-chunk ``(Aqk, A, w_pseudo, u, kg, qg, gc_last)`` of q, k, b, g
    [B, T, H, K], v, w [B, T, H, V]: Aqk, A [B, H, NT, 64, 64], w_pseudo, kg,
    qg [B, H, NT, 64, K], u [B, H, NT, 64, V], gc_last [B, H, NT, K]."""
    _g._check_inputs(q, k, v, w, b, g)
    q, k, v, w, b, g = (t.contiguous() for t in (q, k, v, w, b, g))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // BT
    args = _g.make_args(q, v, scale, chunk=BT)
    dt, dev = q.dtype, q.device
    Aqk = torch.empty(B, H, NT, BT, BT, dtype=dt, device=dev)
    A = torch.empty(B, H, NT, BT, BT, dtype=dt, device=dev)
    wp, kg, qg = (torch.empty(B, H, NT, BT, K, dtype=dt, device=dev) for _ in range(3))
    u = torch.empty(B, H, NT, BT, V, dtype=dt, device=dev)
    gl = torch.empty(B, H, NT, K, dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.load().atomic_gdn2_chunk_wy(ctypes.byref(args), p(q), p(k), p(v), p(w), p(b), p(g), p(Aqk), p(A),
                                          p(wp), p(u), p(kg), p(qg), p(gl), _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_chunk_wy")
    return Aqk, A, wp, u, kg, qg, gl


def _combine_args(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0):
    B, H, NT, C, K = w_pseudo.shape
    V = u.shape[-1]
    if C not in (BT, REF_BLOCK):
        raise _lib.AtomicError(f"gdn2_inter_chunk_combine: blocks of {C} rows (takes {REF_BLOCK} or {BT})")
    dt = w_pseudo.dtype
    if C == REF_BLOCK and dt != torch.float32:
        raise TypeError("the 256-row combine takes the float32 arrays of kernels A and C")
    for t in (Aqk, w_pseudo, u, kg, qg):
        if t.dtype != dt or not t.is_cuda:
            raise TypeError("per-chunk arrays must share one dtype and live on the device")
    if Aqk.shape != (B, H, NT, C, C) or u.shape[:4] != (B, H, NT, C) or kg.shape != w_pseudo.shape \
            or qg.shape != w_pseudo.shape or gc_last.shape != (B, H, NT, K):
        raise ValueError("inconsistent per-chunk array shapes")
    arrays = [t.contiguous() for t in (Aqk, w_pseudo, u, kg, qg)] + [gc_last.to(torch.float32).contiguous()]
    args = _lib.Gdn2Args(B, NT * C, H, K, V, C, _g._DT[dt], _g._DT[dt], float(scale), 0, None, None)
    if h0 is not None:
        h0 = h0.to(torch.float32).contiguous()
    dev = w_pseudo.device
    o = torch.empty(B, H, NT, C, V, dtype=torch.float32, device=dev)
    h_final = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    return args, arrays, h0, o, h_final


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def gdn2_inter_chunk_combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None, debug_tag=""):
    """Kernel D over per-chunk arrays (see ``build_chunk_wy``); h0 [B, H, K, V]
    (sanitised like the reference's ``_sanitize_h0``) or None.  Returns o
    [B, H, NT, BT, V] float32 and h_final [B, H, K, V] float32."""
    args, arrays, h0, o, h_final = _combine_args(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0)
    rc = _lib.load().atomic_gdn2_inter_chunk_combine(ctypes.byref(args), *map(_p, arrays), _p(h0), _p(o),
                                                     _p(h_final), _g._stream(o.device))
    _lib.check(rc, "atomic_gdn2_inter_chunk_combine")
    return o, h_final


def gdn2_inter_chunk_combine_with_state(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None, debug_tag=""):
    """Kernel D that also returns the states of the scan
    (kernel_d_pipeline.py:127-158): ``(o, h_final, h_pre_all, v_new_all)``
    with h_pre_all [NT, B, H, K, V] (the state entering each chunk) and
    v_new_all [NT, B, H, BT, V] in the reference's scan order, float32.  At
    256-row blocks the library writes them in float32 as [B, H, NT, ...]; at
    64-row chunks in the arrays' dtype, transposed.  They are laid out here."""
    args, arrays, h0, o, h_final = _combine_args(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0)
    B, H, NT, C, K = w_pseudo.shape
    V = u.shape[-1]
    dt, dev = w_pseudo.dtype, w_pseudo.device
    if C == REF_BLOCK:
        h_pre = torch.empty(B, H, NT, K, V, dtype=dt, device=dev)
        v_new = torch.empty(B, H, NT, C, V, dtype=dt, device=dev)
    else:
        h_pre = torch.empty(B, H, NT, V, K, dtype=dt, device=dev)
        v_new = torch.empty(B, H, NT, V, C, dtype=dt, device=dev)
    rc = _lib.load().atomic_gdn2_inter_chunk_combine_with_state(
        ctypes.byref(args), *map(_p, arrays), _p(h0), _p(o), _p(h_final), _p(h_pre), _p(v_new),
        _g._stream(dev))
    _lib.check(rc, "atomic_gdn2_inter_chunk_combine_with_state")
    if C != REF_BLOCK:
        h_pre, v_new = h_pre.transpose(-1, -2), v_new.transpose(-1, -2)
    h_pre_all = h_pre.permute(2, 0, 1, 3, 4).to(torch.float32)
    v_new_all = v_new.permute(2, 0, 1, 3, 4).to(torch.float32)
    return o, h_final, h_pre_all, v_new_all


def gdn2_pallas_forward_with_residuals(q, k, v, w, b, g, scale, h0=None, debug_tag="", *, block=REF_BLOCK):
    """The staged forward keeping the backward's residuals
    (kernel_d_pipeline.py:199-228): ``(o [B, T, H, V], h_final, residuals)``
    with residuals Aqk, Akk, A, h_pre_all, v_new_all, w_pseudo, u, kg, qg,
    gc_last, from kernels A, B, C and D run one by one at ``block`` rows (the
    reference's 256, or this library's 64)."""
    from .kernel_a_scores import build_chunk_scores_pallas
    from .kernel_b_solve import wy_solve_pallas
    from .kernel_c_recompute import recompute_wy_pallas
    check_block(block)
    B, T, H, K = q.shape
    V = v.shape[-1]
    Aqk, Akk = build_chunk_scores_pallas(q, k, b, g, scale, block=block)
    A = wy_solve_pallas(Akk)
    w_pseudo, u, kg, qg, gc_last = recompute_wy_pallas(q, k, v, w, b, g, A)
    o_chunks, h_final, h_pre_all, v_new_all = gdn2_inter_chunk_combine_with_state(
        Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=h0)
    o = o_chunks.permute(0, 2, 3, 1, 4).reshape(B, T, H, V)
    residuals = dict(Aqk=Aqk, Akk=Akk, A=A, h_pre_all=h_pre_all, v_new_all=v_new_all, w_pseudo=w_pseudo,
                     u=u, kg=kg, qg=qg, gc_last=gc_last)
    return o, h_final, residuals
