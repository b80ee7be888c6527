"""Mamba2 MB4 (mirror of reference atomic_ops/mamba2_bwd_a_dA_reference.py).

``mamba2_dA_backward(dt_pallas, A, dcumdecay_combined, chunk_size)`` keeps the
reference signature (mamba2_bwd_a_dA_reference.py:60) and returns
``(ddt_contrib2, dA)``: M2's adjoint, the combined cumdecay cotangent masked
by cumdecay's own clip, reverse-cumsummed over the chunk and masked by the
step exponent's clip, times A (ddt's second part, dt_pallas's layout) and
times dt summed over everything but the head (dA), each sanitised (:89-113).
dt_pallas [B, H, NT, C, P] bf16 or float32, A [H], dcumdecay_combined
float32.  ``reshape_dt_to_pallas`` / ``unreshape_dt_from_pallas`` are the
reference's layout helpers (:118-140).  Every computation runs in
libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m
from .kernel_mamba2_a_decay import _ptr


def reshape_dt_to_pallas(dt, chunk_size):
    """(B, L, H, P) -> (B, H, NT, C, P)."""
    b, l, h, p = dt.shape
    return dt.reshape(b, l // chunk_size, chunk_size, h, p).permute(0, 3, 1, 2, 4)


def unreshape_dt_from_pallas(t):
    """(B, H, NT, C, P) -> (B, L, H, P)."""
    b, h, nt, c, p = t.shape
    return t.permute(0, 2, 3, 1, 4).reshape(b, nt * c, h, p)


def mamba2_dA_backward(dt_pallas, A, dcumdecay_combined, chunk_size):
    if dt_pallas.dim() != 5 or not dt_pallas.is_cuda or dt_pallas.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("dt_pallas must be a bf16 / float32 device tensor [B, H, NT, C, P]")
    b, h, nt, c, p = dt_pallas.shape
    if c != chunk_size:                                                   # :84
        raise ValueError(f"dt_pallas's chunk {c} is not chunk_size={chunk_size}")
    if A.shape != (h,) or dcumdecay_combined.shape != dt_pallas.shape:
        raise ValueError("A must be (H,) and dcumdecay_combined shaped like dt_pallas")
    dtp = dt_pallas.contiguous()
    A = A.to(torch.float32).contiguous()
    dcum = dcumdecay_combined.to(torch.float32).contiguous()
    dtype = _lib.ATOMIC_BF16 if dtp.dtype == torch.bfloat16 else _lib.ATOMIC_F32
    args = _lib.Mamba2Args(b, nt * c, h, p, 128, c, dtype, dtype, 0)
    lib = _lib.load()
    nws = lib.atomic_mamba2_da_backward_workspace_size(ctypes.byref(args))
    if nws == 0:
        raise _lib.AtomicError("atomic_mamba2_da_backward_workspace_size: unsupported shape")
    dev = dtp.device
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    ddt2 = torch.empty(dtp.shape, dtype=torch.float32, device=dev)
    dA = torch.empty(h, dtype=torch.float32, device=dev)
    rc = lib.atomic_mamba2_da_backward(ctypes.byref(args), _ptr(dtp), _ptr(A), _ptr(dcum), _ptr(ddt2), _ptr(dA),
                                       _ptr(ws), ctypes.c_size_t(ws.numel()), _m._stream(dev))
    _lib.check(rc, "atomic_mamba2_da_backward")
    return ddt2, dA
