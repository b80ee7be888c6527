"""Kernel B alone (mirror of reference atomic_ops/kernel_b_solve.py).

``wy_solve_pallas(Akk)`` keeps the reference signature (kernel_b_solve.py:151)
and returns A = (I + Akk)^-1 per chunk, ``[B, H, NT, BT, BT]`` in Akk's
dtype, by forward substitution on 16-row diagonal blocks and block products
below them (the reference's MB = 16 block recursion); only the strictly
lower blocks of Akk are read, as in the reference.  BT is 64 here.  Every
computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT


def wy_solve_pallas(Akk):
    if not Akk.is_cuda or Akk.dtype not in _g._DT:
        raise TypeError("Akk must be a bf16 or fp32 device tensor")
    if Akk.dim() != 5 or Akk.shape[-2:] != (BT, BT):
        raise ValueError(f"Akk must be [B, H, NT, {BT}, {BT}], got {tuple(Akk.shape)}")
    Akk = Akk.contiguous()
    B, H, NT = Akk.shape[:3]
    # K = V = 64 only sizes the launch; the solve reads nothing else
    args = _lib.Gdn2Args(B, NT * BT, H, 64, 64, BT, _g._DT[Akk.dtype], _g._DT[Akk.dtype], 1.0, 0, None, None)
    A = torch.empty_like(Akk)
    rc = _lib.load().atomic_gdn2_wy_solve(ctypes.byref(args), ctypes.c_void_p(Akk.data_ptr()),
                                          ctypes.c_void_p(A.data_ptr()), _g._stream(Akk.device))
    _lib.check(rc, "atomic_gdn2_wy_solve")
    return A
