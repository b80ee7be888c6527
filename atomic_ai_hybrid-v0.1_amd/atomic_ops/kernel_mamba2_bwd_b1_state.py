"""Mamba2 MB1 + MB3 (mirror of reference atomic_ops/kernel_mamba2_bwd_b1_state.py).

``mamba2_bwd_scan(dt, A, B, C, x, chunk_size, do, dstate_final, state0=None,
interpret=False)`` keeps the reference signature (kernel_mamba2_bwd_b1_state.py:132)
and returns ``(ddt, dB, dC, dx, dstate0, dcumdecay)``: M2's cumdecay, the
reference chunk's forward re-run for the state entering each chunk, the
state-only reverse scan whose sanitised carries are MB2's dstate_end_grad,
MB2 and the sanitised sums of the two halves (:168-256).  As in the reference,
ddt is only the dt x part and dcumdecay [B, H, NT, C, P] is both halves' sum,
for ``mamba2_dA_backward`` (MB4).  dt, x, B, C bfloat16 or float32
(one dtype), do bf16 or float32, A, dstate_final, state0 float32; the
results are float32.  Every computation runs in libatomic_hybrid.so; there is
no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import mamba2 as _m
from .kernel_mamba2_a_decay import _ptr, stage_args


def mamba2_bwd_scan(dt, A, B, C, x, chunk_size, do, dstate_final, state0=None, interpret=False):
    b, l, h, p = dt.shape
    n = B.shape[-1]
    if l % chunk_size != 0:
        raise ValueError(f"seq_len={l} must be divisible by chunk_size={chunk_size}.")   # :160
    nt = l // chunk_size
    if x.shape != dt.shape or x.dtype != dt.dtype or B.shape != (b, l, n) or C.shape != B.shape \
            or B.dtype != dt.dtype or C.dtype != dt.dtype:
        raise ValueError("x must match dt; B and C must be [B, T, N] in dt's dtype")
    if do.shape != dt.shape or do.dtype not in (torch.bfloat16, torch.float32) or not do.is_cuda:
        raise ValueError("do must be a bf16 / float32 device tensor of dt's shape")
    if A.shape != (h,):
        raise ValueError(f"A must be (n_heads_ssm,)={h}, got {tuple(A.shape)}")
    for name, t in (("dstate_final", dstate_final), ("state0", state0)):
        if t is not None and t.shape != (b, h, p, n):
            raise ValueError(f"{name} must be [B, H, P, N]")
    args = stage_args(dt, n, chunk_size)
    args.dy_dtype = _lib.ATOMIC_BF16 if do.dtype == torch.bfloat16 else _lib.ATOMIC_F32
    dt, x, B, C, do = (t.contiguous() for t in (dt, x, B, C, do))
    A = A.to(torch.float32).contiguous()
    dsf = None if dstate_final is None else dstate_final.to(torch.float32).contiguous()
    s0 = None if state0 is None else state0.to(torch.float32).contiguous()
    lib = _lib.load()
    nws = lib.atomic_mamba2_bwd_scan_workspace_size(ctypes.byref(args))
    if nws == 0:
        raise _lib.AtomicError("atomic_mamba2_bwd_scan_workspace_size: unsupported shape")
    dev = dt.device
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    ddt, dx = torch.empty(b, l, h, p, **f32), torch.empty(b, l, h, p, **f32)
    dB, dC = torch.empty(b, l, n, **f32), torch.empty(b, l, n, **f32)
    dstate0 = torch.empty(b, h, p, n, **f32)
    dcum = torch.empty(b, h, nt, chunk_size, p, **f32)
    rc = lib.atomic_mamba2_bwd_scan(ctypes.byref(args), _ptr(dt), _ptr(A), _ptr(B), _ptr(C), _ptr(x), _ptr(do),
                                    _ptr(dsf), _ptr(s0), _ptr(ddt), _ptr(dB), _ptr(dC), _ptr(dx), _ptr(dstate0),
                                    _ptr(dcum), _ptr(ws), ctypes.c_size_t(ws.numel()), _m._stream(dev))
    _lib.check(rc, "atomic_mamba2_bwd_scan")
    return ddt, dB, dC, dx, dstate0, dcum
