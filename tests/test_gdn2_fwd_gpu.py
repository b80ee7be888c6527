"""GDN2 forward on the GPU (through the C ABI) against the CPU oracle."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import gdn2 as G
from atomic_ops import inputs
from oracle import gdn2 as og

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16


def _run(B, T, H, K, dtype, seed, scale=1.0, g_mean=3.0, h0=False, mutate=None):
    inp = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype, g_mean=g_mean)
    if mutate:
        mutate(inp)
    q, k, v, w, b, g = (inp[n] for n in "q k v w b g".split())
    hz = None
    if h0:
        hz = 0.3 * torch.randn(B, H, K, K, generator=torch.Generator().manual_seed(seed + 1))
    o_ref, h_ref = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 64, h0=hz)
    dev = [t.cuda() for t in (q, k, v, w, b, g)]
    o, hf, ws = G.forward(*dev, scale, h0=hz.cuda() if hz is not None else None, save=True)
    torch.cuda.synchronize()
    return (q, k, v, w, b, g, hz), (o, hf, ws), (o_ref, h_ref)


@pytest.mark.parametrize("B,T,H,K,dtype,scale,h0", [
    (1, 512, 4, 64, F32, 1.0, False),        # config 0
    (1, 256, 2, 64, F32, 0.125, True),
    (2, 256, 2, 128, BF16, 1.0, False),      # config 2 head shape
    (1, 192, 3, 128, BF16, 128 ** -0.5, True),
    (1, 128, 2, 128, F32, 1.0, False),
    (2, 128, 2, 64, BF16, 1.0, False),
    (1, 64, 2, 128, BF16, 1.0, True),        # one chunk: only the state loop's tail step
    (1, 128, 48, 128, BF16, 1.0, True),      # 48 heads: 32-column V tiles (fewer heads take 16)
])
def test_forward_matches_oracle(B, T, H, K, dtype, scale, h0):
    banner(f"gdn2 fwd B{B} T{T} H{H} K{K} {dtype} scale={scale} h0={h0}")
    _, (o, hf, _), (o_ref, h_ref) = _run(B, T, H, K, dtype, seed=B * 100 + K, scale=scale, h0=h0)
    eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
    print(f"  rel_err o={eo:.3e} h_final={eh:.3e}")
    assert torch.isfinite(o).all() and torch.isfinite(hf).all()
    assert eo < tol_for(dtype)
    assert eh < tol_for(dtype)


@pytest.mark.parametrize("dtype,K", [(F32, 64), (BF16, 128)])
def test_chunk_intermediates_match_oracle(dtype, K):
    """Stage-level check of the intra-chunk kernel (A, B, C of the reference
    pipeline) and the saved per-chunk state / v_new of the state kernel."""
    B, T, H = 1, 192, 2
    banner(f"gdn2 stages {dtype} K{K}")
    (q, k, v, w, b, g, _), (o, hf, ws), _ = _run(B, T, H, K, dtype, seed=7)
    args = G.make_args(q, v, 1.0)
    views = G.chunk_views(ws, args)
    _, _, stages = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 64, return_stages=True)
    tol = tol_for(dtype)
    for n, st in enumerate(stages):
        for name, ref in (("qg", st["qg"]), ("kg", st["kg"]), ("w_pseudo", st["w_pseudo"]),
                          ("u", st["u"]), ("aqk", st["Aqk"]), ("ainv", st["A"]),
                          ("gc_last", st["gc_last"])):
            got = views[name][:, :, n]
            e = rel_err(got, ref)
            assert e < tol, (n, name, e)
        e = rel_err(views["h_pre_t"][:, :, n].transpose(-1, -2), st["h_pre"]) if n else 0.0
        assert e < tol, (n, "h_pre", e)
        e = rel_err(views["v_new_t"][:, :, n].transpose(-1, -2), st["v_new"])
        assert e < tol, (n, "v_new", e)


@pytest.mark.parametrize("case,dtype,K", [
    ("positive_gate", F32, 64), ("deep_decay", F32, 64),
    ("positive_gate", BF16, 128), ("deep_decay", BF16, 128),
    ("deep_decay_upper_columns", BF16, 128),
])
def test_exact_pairwise_path(case, dtype, K):
    """Chunks where the factorised scores could overflow (or a gate is
    positive) take the exact pairwise path; results still match the oracle,
    including the reference's +-20 clip on the pairwise decay.  In the last
    case only columns 64..127 of chunk 1 decay past the bound."""
    banner(f"gdn2 exact path {case} {dtype} K{K}")

    def mutate(inp):
        g = inp["g"]
        if case == "positive_gate":
            g[:, 5:9] = 0.4           # breaks monotone decay in chunk 0
        elif case == "deep_decay":
            g[:, 64:128] *= 40.0      # ~-2 per step: chunk 1 decays past -64
        else:
            g[:, 64:128, :, 64:] *= 40.0
    _, (o, hf, _), (o_ref, h_ref) = _run(1, 192, 2, K, dtype, seed=11, mutate=mutate)
    eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
    print(f"  rel_err o={eo:.3e} h_final={eh:.3e}")
    assert eo < tol_for(dtype) and eh < tol_for(dtype)


def test_rejects_bad_shapes():
    q = torch.zeros(1, 100, 1, 64, device="cuda")
    v = torch.zeros(1, 100, 1, 64, device="cuda")
    with pytest.raises(ValueError):
        G.forward(q, q, v, v, q, q, 1.0)
