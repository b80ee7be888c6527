"""atomic_gdn2_fwd_noalloc, the forward that allocates nothing (its scratch
is the library's fixed device array), against atomic_gdn2_fwd on the same
inputs: two calls in a row, the second with a smaller input, each into
NaN-filled outputs (every element must be written)."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import _lib
from atomic_ops import gdn2 as G
from atomic_ops import inputs
from oracle import gdn2 as og

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32
# bf16 B2 T4096 H16: 64 chunks per batch row, more than the 49-chunk window
# that fits the scratch at 16 heads, so the state crosses a window boundary
CASES = [(2, 4096, 16, 128, BF16, True), (1, 512, 4, 64, F32, False)]


def _nan_outputs(B, T, H, K):
    nan = float("nan")
    return (torch.full((B, T, H, K), nan, device="cuda"), torch.full((B, H, K, K), nan, device="cuda"))


def test_noalloc_matches_workspace_forward_two_calls():
    for B, T, H, K, dtype, with_h0 in CASES:
        banner(f"gdn2 fwd noalloc B{B} T{T} H{H} K{K} {dtype} h0={with_h0}")
        cpu = inputs.gdn2_inputs(B, T, H, K, K, seed=T + H, dtype=dtype)
        h0 = 0.3 * torch.randn(B, H, K, K, generator=torch.Generator().manual_seed(5)) if with_h0 else None
        dev = [cpu[n].cuda() for n in ("q", "k", "v", "w", "b", "g")]
        h0d = h0.cuda() if h0 is not None else None
        o_ref, h_ref, _ = G.forward(*dev, 1.0, h0=h0d)
        o, hf = _nan_outputs(B, T, H, K)
        G.forward_noalloc(*dev, 1.0, h0=h0d, o=o, h_final=hf)
        torch.cuda.synchronize()
        assert torch.isfinite(o).all() and torch.isfinite(hf).all()
        eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
        print(f"  against atomic_gdn2_fwd: o={eo:.2e} h_final={eh:.2e}", flush=True)
        assert eo <= 1e-6 and eh <= 1e-6
        if T <= 512:
            q, k, v, w, b, g = (cpu[n] for n in ("q", "k", "v", "w", "b", "g"))
            o_or, h_or = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 64, h0=h0)
            assert rel_err(o, o_or) < tol_for(dtype) and rel_err(hf, h_or) < tol_for(dtype)


def test_noalloc_rejects_what_does_not_fit():
    banner("gdn2 fwd noalloc rejections")
    # 1024 heads: one chunk of intermediates plus two states exceeds the scratch
    d = inputs.gdn2_inputs(1, 64, 1024, 128, 128, seed=1, dtype=BF16, device="cuda")
    dev = [d[n] for n in ("q", "k", "v", "w", "b", "g")]
    with pytest.raises(_lib.AtomicError, match="SCRATCH"):
        G.forward_noalloc(*dev, 1.0)
    # SAVE asks for intermediates that outlive the call
    import ctypes
    small = inputs.gdn2_inputs(1, 64, 2, 64, 64, seed=2, dtype=F32, device="cuda")
    q, k, v, w, b, g = (small[n] for n in ("q", "k", "v", "w", "b", "g"))
    args = G.make_args(q, v, 1.0, flags=_lib.GDN2_SAVE)
    o = torch.empty(1, 64, 2, 64, device="cuda")
    hf = torch.empty(1, 2, 64, 64, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.load().atomic_gdn2_fwd_noalloc(ctypes.byref(args), p(q), p(k), p(v), p(w), p(b), p(g), None,
                                             p(o), p(hf), None)
    assert rc == -6
