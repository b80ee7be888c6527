"""Drop-in trainable Mamba2 SSD op (mirror of reference
atomic_ops/kernel_mamba2_trainable_B6.py).

``mamba2_pallas_forward_trainable_B6(dt, x, B, C, A, chunk_size, state0=None)``
keeps the reference signature (kernel_mamba2_trainable_B6.py:137-155) and
returns ``(y, state_final)``; its backward returns ``(ddt, dx, dB, dC, dA,
dstate0)`` cast to the primals' dtypes after the final clip(+-1e4) /
nan_to_num (kernel_mamba2_trainable_B6.py:108-131).  ``chunk_size`` is not
differentiable (:72).  The forward keeps the per-chunk states for the
backward instead of re-running the forward scan.  state0 is clipped to +-1e4
and nan_to_num'd first, as in the reference's staged forward
(kernel_mamba2_c_interchunk.py:56-58); dstate0 is the gradient at the
sanitised state0.
"""
from __future__ import annotations

import torch

from . import _lib
from . import mamba2 as _m


class _Mamba2Core(torch.autograd.Function):
    @staticmethod
    def forward(ctx, dt, x, B, C, A, chunk_size, state0):
        need = any(ctx.needs_input_grad)
        ctx.A_dtype, ctx.state0_dtype = A.dtype, state0.dtype
        # the tensors the library sees (row-strided views as they are, other
        # layouts as dense copies), kept for the backward: its reuse of the
        # forward's workspace is checked against these addresses and strides
        dt, x, B, C = (_lib.row_view(t)[0] for t in (dt, x, B, C))
        A = A.to(torch.float32).contiguous()
        state0 = state0.to(torch.float32).contiguous()
        # state0 is sanitised first, as the reference's staged forward does
        # (mamba2_pallas_forward -> mamba2_inter_chunk_combine,
        # kernel_mamba2_c_interchunk.py:56-58)
        y, state_final, ws = _m.forward(dt, x, B, C, A, chunk_size, state0, save=need, sanitize_state0=True)
        if need:
            ctx.save_for_backward(dt, x, B, C, A, state0)
            ctx.ws = ws
            ctx.chunk_size = chunk_size
        return y, state_final

    @staticmethod
    def backward(ctx, dy, dstate_final):
        dt, x, B, C, A, state0 = ctx.saved_tensors
        # The first backward reuses the forward's per-chunk states and releases
        # them; a further backward (retain_graph) recomputes them.
        ws, ctx.ws = ctx.ws, None
        call = lambda reuse: _m.backward(dt, x, B, C, A, ctx.chunk_size, dy, dstate_final=dstate_final,
                                         state0=state0, workspace=ws, reuse=reuse, sanitize_state0=True)
        try:
            ddt, dx, dB, dC, dA, dstate0 = call(ws is not None)
        except _lib.AtomicError as e:
            if e.code != _lib.ATOMIC_ERR_REUSE:
                raise
            # the library no longer holds the record of the saving forward
            # (e.g. evicted): recompute it instead, which gives the same gradients
            ddt, dx, dB, dC, dA, dstate0 = call(False)
        return ddt, dx, dB, dC, dA.to(ctx.A_dtype), None, dstate0.to(ctx.state0_dtype)


def mamba2_pallas_forward_trainable_B6(dt, x, B, C, A, chunk_size, state0=None):
    """dt, x: [b, l, h, p]; B, C: [b, l, n]; A: [h] float32; state0: [b, h, p, n]
    float32 (zeros when None).  Returns y [b, l, h, p] float32 and
    state_final [b, h, p, n] float32."""
    b, l, h, p = dt.shape
    if state0 is None:
        state0 = torch.zeros(b, h, p, B.shape[-1], dtype=torch.float32, device=dt.device)
    return _Mamba2Core.apply(dt, x, B, C, A, chunk_size, state0)


def mamba2_pallas_forward(dt, x, B, C, A, chunk_size, state0=None):
    """Forward only (reference kernel_mamba2_c_interchunk.py:90-100), state0
    sanitised first like the reference's combine (:56-58)."""
    y, state_final, _ = _m.forward(dt, x, B, C, A, chunk_size, state0, sanitize_state0=True)
    return y, state_final
