"""Kernel B alone (mirror of reference atomic_ops/kernel_b_solve.py).

``wy_solve_pallas(Akk)`` keeps the reference signature (kernel_b_solve.py:151)
and returns A = (I + Akk)^-1 per block.  For the reference's float32
``[B, H, NT, 256, 256]`` blocks it follows kernel_b_solve.py:68-148: each
128-row half by forward substitution on 16-row diagonal blocks and the block
recursion below them, then A10 = -A11 T10 A00, sanitising (clip +-1e4,
nan_to_num) at every block product as the reference does.  For this
library's ``[..., 64, 64]`` blocks (bf16 or fp32) it runs the 64-row solve of
the whole path, which clips once at the end.  Only the strictly lower part
of Akk is read, as in the reference.  Every computation runs in
libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT, RUN_BLOCK


def wy_solve_pallas(Akk):
    if not Akk.is_cuda or Akk.dtype not in _g._DT:
        raise TypeError("Akk must be a bf16 or fp32 device tensor")
    blk = Akk.shape[-1]
    if Akk.dim() != 5 or Akk.shape[-2] != blk or blk not in (BT, RUN_BLOCK):
        raise ValueError(f"Akk must be [B, H, NT, {BT}, {BT}] (or {RUN_BLOCK} x {RUN_BLOCK}), "
                         f"got {tuple(Akk.shape)}")
    if blk == BT and Akk.dtype != torch.float32:
        raise TypeError("the 256-row solve takes the float32 Akk of kernel A")
    Akk = Akk.contiguous()
    B, H, NT = Akk.shape[:3]
    # K = V = 64 only sizes the plan; the solve reads nothing else
    args = _lib.Gdn2Args(B, NT * blk, H, 64, 64, blk, _g._DT[Akk.dtype], _g._DT[Akk.dtype], 1.0, 0, None, None)
    A = torch.empty_like(Akk)
    rc = _lib.load().atomic_gdn2_wy_solve(ctypes.byref(args), ctypes.c_void_p(Akk.data_ptr()),
                                          ctypes.c_void_p(A.data_ptr()), _g._stream(Akk.device))
    _lib.check(rc, "atomic_gdn2_wy_solve")
    return A
