"""Shared checks of the GDN2 backward stage mirrors (per-block arrays at the
reference's 256-row block, kernel_a_scores.py:15-17)."""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import gdn2 as _g
from .kernel_a_scores import BT


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def blocks_f32(name, t, shape):
    """A float32 per-block device array of exactly ``shape``, contiguous."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32:
        raise TypeError(f"{name} must be a float32 device tensor")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def operand(name, t, shape, dtype=None):
    """A bf16 or float32 device array of ``shape`` (and ``dtype`` when given)."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype not in _g._DT:
        raise TypeError(f"{name} must be a bf16 or float32 device tensor")
    if tuple(t.shape) != tuple(shape) or (dtype is not None and t.dtype != dtype):
        raise ValueError(f"{name} must be {tuple(shape)}" + (f" in {dtype}" if dtype is not None else ""))
    return t.contiguous()


def block_args(B, H, NT, K, V, dtype, do_dtype, scale):
    if K not in (64, 128) or V != K:
        raise ValueError("the head dims must be K = V in {64, 128}")
    return _lib.Gdn2Args(B, NT * BT, H, K, V, BT, _g._DT[dtype], _g._DT[do_dtype], float(scale), 0)
