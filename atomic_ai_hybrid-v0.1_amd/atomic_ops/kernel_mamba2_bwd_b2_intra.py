"""Mamba2 stage MB2 (mirror of reference atomic_ops/kernel_mamba2_bwd_b2_intra.py).

``intra_chunk_ssd_bwd_pallas(dt, x, B, C, cumdecay, dy, dstate_end_grad,
chunk_size, interpret=False)`` keeps the reference signature
(kernel_mamba2_bwd_b2_intra.py:130) and returns ``(ddt, dx, dB, dC, dcum)``:
the backward of M3 per (batch, head, chunk) with the state-end part as
whole-chunk products (:53-66), the y_diag part over min(128, chunk_size)-row
sub-block pairs with a sanitise after every accumulation (:73-113), and the
per-head dB, dC summed over the heads (:168-178).  dt, x, B, C are bfloat16
or float32 (one dtype), dy bf16 or float32, cumdecay
[B, H, NT, C, P] and dstate_end_grad [B, H, NT, P, N] float32.  Returns float32
ddt, dx [B, T, H, P], dB, dC [B, T, N] and dcum [B, H, NT, C, P].  Every
computation runs in libatomic_hybrid.so; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m
from .kernel_mamba2_a_decay import _ptr, stage_args


def intra_chunk_ssd_bwd_pallas(dt, x, B, C, cumdecay, dy, dstate_end_grad, chunk_size, interpret=False):
    b, l, h, p = dt.shape
    n = B.shape[-1]
    if l % chunk_size != 0:
        raise ValueError(f"seq_len={l} must be divisible by chunk_size={chunk_size}")   # :132
    nt = l // chunk_size
    if x.shape != dt.shape or x.dtype != dt.dtype or B.shape != (b, l, n) or C.shape != B.shape \
            or B.dtype != dt.dtype or C.dtype != dt.dtype:
        raise ValueError("x must match dt; B and C must be [B, T, N] in dt's dtype")
    if dy.shape != dt.shape or dy.dtype not in (torch.bfloat16, torch.float32) or not dy.is_cuda:
        raise ValueError("dy must be a bf16 / float32 device tensor of dt's shape")
    if cumdecay.shape != (b, h, nt, chunk_size, p):
        raise ValueError(f"cumdecay must be [B, H, NT, {chunk_size}, P], got {tuple(cumdecay.shape)}")
    if dstate_end_grad.shape != (b, h, nt, p, n):
        raise ValueError(f"dstate_end_grad must be [B, H, NT, P, N], got {tuple(dstate_end_grad.shape)}")
    args = stage_args(dt, n, chunk_size)
    args.dy_dtype = _lib.ATOMIC_BF16 if dy.dtype == torch.bfloat16 else _lib.ATOMIC_F32
    dt, x, B, C, dy = (t.contiguous() for t in (dt, x, B, C, dy))
    cum = cumdecay.to(torch.float32).contiguous()
    dse = dstate_end_grad.to(torch.float32).contiguous()
    lib = _lib.load()
    nws = lib.atomic_mamba2_intra_chunk_ssd_bwd_workspace_size(ctypes.byref(args))
    if nws == 0:
        raise _lib.AtomicError("atomic_mamba2_intra_chunk_ssd_bwd_workspace_size: unsupported shape")
    dev = dt.device
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    ddt = torch.empty(b, l, h, p, dtype=torch.float32, device=dev)
    dx = torch.empty_like(ddt)
    dB = torch.empty(b, l, n, dtype=torch.float32, device=dev)
    dC = torch.empty_like(dB)
    dcum = torch.empty(b, h, nt, chunk_size, p, dtype=torch.float32, device=dev)
    rc = lib.atomic_mamba2_intra_chunk_ssd_bwd(ctypes.byref(args), _ptr(dt), _ptr(x), _ptr(B), _ptr(C), _ptr(cum),
                                               _ptr(dy), _ptr(dse), _ptr(ddt), _ptr(dx), _ptr(dB), _ptr(dC),
                                               _ptr(dcum), _ptr(ws), ctypes.c_size_t(ws.numel()),
                                               _m._stream(dev))
    _lib.check(rc, "atomic_mamba2_intra_chunk_ssd_bwd")
    return ddt, dx, dB, dC, dcum
