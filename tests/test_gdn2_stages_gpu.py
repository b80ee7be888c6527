"""Stage-level GDN2 forward through the C ABI: kernels A + B + C
(``build_chunk_wy``) and kernel D (``gdn2_inter_chunk_combine``,
kernel_d_pipeline.py:94-124) over per-chunk arrays in the reference's layout.
Against the oracle's stages and its restatement of the combine, and the two
stages chained against the whole-path forward."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import _lib, inputs
from atomic_ops import gdn2 as G
from atomic_ops import kernel_d_pipeline as KD
from oracle import gdn2 as og

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
STAGES = ("Aqk", "A", "w_pseudo", "u", "kg", "qg", "gc_last")


def _inputs(B, T, H, K, dtype, seed):
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype)
    return [d[n] for n in ("q", "k", "v", "w", "b", "g")]


@pytest.mark.parametrize("dtype,K", [(F32, 64), (F32, 128), (BF16, 128)])
def test_stages_match_the_oracle(dtype, K):
    B, T, H = 1, 192, 2
    banner(f"gdn2 stage entries {dtype} K{K}")
    q, k, v, w, b, g = _inputs(B, T, H, K, dtype, 51 + K)
    gen = torch.Generator().manual_seed(52)
    h0 = 0.5 * torch.randn(B, H, K, K, generator=gen)
    h0[0, 0, 0, 0], h0[0, 1, 1, 1] = float("nan"), 3e4          # sanitised by the combine
    _, _, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 0.8, 64, return_stages=True)
    ref = {n: torch.stack([s[n] for s in st], 2) for n in STAGES}
    got = KD.build_chunk_wy(*(t.cuda() for t in (q, k, v, w, b, g)), 0.8)
    tol = tol_for(dtype)
    for name, t in zip(STAGES, got):
        e = rel_err(t, ref[name])
        print(f"  {name}: rel_err {e:.2e}")
        assert t.shape == ref[name].shape and e < tol, name
    # kernel D on the oracle's own stages, against the oracle's combine
    o_ref, h_ref = og.gdn2_inter_chunk_combine(*(ref[n] for n in ("Aqk", "w_pseudo", "u", "kg", "qg", "gc_last")),
                                               0.8, h0=h0)
    args = [ref[n].to(dtype).cuda() for n in ("Aqk", "w_pseudo", "u", "kg", "qg")] + [ref["gc_last"].float().cuda()]
    o, hf = KD.gdn2_inter_chunk_combine(*args, 0.8, h0=h0.cuda())
    torch.cuda.synchronize()
    eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
    print(f"  combine: o {eo:.2e} h_final {eh:.2e}")
    assert o.shape == o_ref.shape and eo < tol and eh < tol


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_chained_stages_equal_the_whole_forward(dtype):
    B, T, H, K = 2, 256, 2, 128
    banner(f"gdn2 chained stages {dtype}")
    q, k, v, w, b, g = (t.cuda() for t in _inputs(B, T, H, K, dtype, 61))
    h0 = 0.3 * torch.randn(B, H, K, K, device="cuda")
    o_w, h_w, _ = G.forward(q, k, v, w, b, g, 1.0, h0=h0)
    Aqk, A, wp, u, kg, qg, gl = KD.build_chunk_wy(q, k, v, w, b, g, 1.0)
    o_c, h_c = KD.gdn2_inter_chunk_combine(Aqk, wp, u, kg, qg, gl, 1.0, h0=h0)
    torch.cuda.synchronize()
    o_c = o_c.permute(0, 2, 3, 1, 4).reshape(B, T, H, K)
    assert torch.equal(o_c, o_w) and torch.equal(h_c, h_w)


def test_stage_entries_reject_other_chunks():
    banner("gdn2 stage chunk check")
    q, k, v, w, b, g = (t.cuda() for t in _inputs(1, 256, 2, 64, F32, 3))
    with pytest.raises(_lib.AtomicError):
        KD.gdn2_inter_chunk_combine(*(torch.zeros(1, 2, 2, 128, n, device="cuda") for n in (128, 64, 64, 64, 64)),
                                    torch.zeros(1, 2, 2, 64, device="cuda"), 1.0)
