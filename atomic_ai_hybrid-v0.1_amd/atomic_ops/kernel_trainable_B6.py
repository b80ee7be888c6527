"""Drop-in trainable GDN2 op (mirror of reference atomic_ops/kernel_trainable_B6.py).

``gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None)`` keeps the
reference signature and argument order (kernel_trainable_B6.py:187-194) and
returns ``(o, h_final)``; its backward returns ``(dq, dk, dv, dw, db, dg, dh0)``
cast to the primals' dtypes after the final clip(+-1e4) / nan_to_num
(kernel_trainable_B6.py:173-181).  ``scale`` is not differentiable
(kernel_trainable_B6.py:86).  h0 is clipped to +-1e4 and nan_to_num'd before
the first chunk, as in the reference's forward (kernel_d_pipeline.py:54-55);
dh0 is the gradient at the sanitised h0.  Forward and backward run in libatomic_hybrid.so;
the forward keeps its per-chunk intermediates for the backward instead of
recomputing them (the reference recomputes; both give the same gradient).
"""
from __future__ import annotations

import os
import sys

import torch

from . import _lib
from . import gdn2 as _g

# The reference's opt-in stage check (GDN2_FWD_DIAG=1, read at import,
# kernel_d_pipeline.py:48-91): every forward then also reduces each stage of
# the pipeline to its non-finite count and max |x| (extra launches; nothing
# extra runs when it is off) and prints the stages that are non-finite or
# above 1e6.
_GDN2_FWD_DIAG = os.environ.get("GDN2_FWD_DIAG", "0") == "1"


def _forward(q, k, v, w, b, g, scale, h0, save, debug_tag=""):
    # h0 is sanitised first, as the reference's staged forward does
    # (gdn2_pallas_forward -> gdn2_inter_chunk_combine, kernel_d_pipeline.py:54-55,101)
    if not _GDN2_FWD_DIAG:
        return _g.forward(q, k, v, w, b, g, scale, h0, save=save, sanitize_h0=True)
    rep = _lib.StageReports(_lib.GDN2_DIAG_STAGES, q.device)
    out = _g.forward(q, k, v, w, b, g, scale, h0, save=save, diag=rep, sanitize_h0=True)
    for line in rep.messages(debug_tag, 0, _lib.GDN2_DIAG_FWD):
        print(line, file=sys.stderr, flush=True)
    return out


class _Gdn2Core(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, w, b, g, scale, h0):
        need = any(ctx.needs_input_grad)
        h0_dtype = h0.dtype
        # the tensors the library sees (row-strided views as they are, other
        # layouts as dense copies), kept for the backward: its reuse of the
        # forward's workspace is checked against these addresses and strides
        q, k, v, w, b, g = (_g.rows(t)[0] for t in (q, k, v, w, b, g))
        h0 = h0.to(torch.float32).contiguous()
        o, h_final, ws = _forward(q, k, v, w, b, g, scale, h0, need)
        if need:
            ctx.save_for_backward(q, k, v, w, b, g, h0)
            ctx.ws = ws
            ctx.scale = scale
            ctx.h0_dtype = h0_dtype
        return o, h_final

    @staticmethod
    def backward(ctx, do, dh_final):
        q, k, v, w, b, g, h0 = ctx.saved_tensors
        # The first backward reuses the forward's intermediates and releases
        # them; a further backward (retain_graph) recomputes the forward into
        # a fresh workspace instead of reading one that holds nothing.
        ws, ctx.ws = ctx.ws, None
        try:
            grads = _g.backward(q, k, v, w, b, g, ctx.scale, do, dh_final=dh_final, h0=h0,
                                workspace=ws, reuse=ws is not None, sanitize_h0=True)
        except _lib.AtomicError as e:
            if e.code != _lib.ATOMIC_ERR_REUSE:
                raise
            # the library no longer holds the record of the saving forward
            # (e.g. evicted): recompute it into the same workspace instead,
            # which gives the same gradients
            grads = _g.backward(q, k, v, w, b, g, ctx.scale, do, dh_final=dh_final, h0=h0,
                                workspace=ws, reuse=False, sanitize_h0=True)
        dq, dk, dv, dw, db, dg, dh0 = grads
        return dq, dk, dv, dw, db, dg, None, dh0.to(ctx.h0_dtype)


def gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None):
    """q, k, b, g: [B, T, H, K]; v, w: [B, T, H, V]; h0: [B, H, K, V] fp32
    (zeros when None).  Returns o [B, T, H, V] fp32 and h_final [B, H, K, V]."""
    B, T, H, K = q.shape
    if h0 is None:
        h0 = torch.zeros(B, H, K, v.shape[-1], dtype=torch.float32, device=q.device)
    return _Gdn2Core.apply(q, k, v, w, b, g, scale, h0)


def gdn2_pallas_forward(q, k, v, w, b, g, scale, h0=None, debug_tag=""):
    """Forward only (reference kernel_d_pipeline.py:161-196); ``debug_tag``
    prefixes the stage reports when GDN2_FWD_DIAG=1."""
    o, h_final, _ = _forward(q, k, v, w, b, g, scale, h0, False, debug_tag)
    return o, h_final
