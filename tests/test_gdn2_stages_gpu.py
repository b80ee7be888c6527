"""Stage-level GDN2 forward through the C ABI: kernels A, B and C alone
(``build_chunk_scores_pallas``, ``wy_solve_pallas``, ``recompute_wy_pallas``,
kernel_a_scores.py:69, kernel_b_solve.py:151, kernel_c_recompute.py:91) and
in one pass (``build_chunk_wy``), and kernel D (``gdn2_inter_chunk_combine``,
kernel_d_pipeline.py:94-124), over per-chunk arrays in the reference's
layout.  Against the oracle's stages and its restatement of the combine, the
stages chained against the whole-path forward, and the solve against the
identity (I + Akk) A = I."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import _lib, inputs
from atomic_ops import gdn2 as G
from atomic_ops import kernel_a_scores as KA
from atomic_ops import kernel_b_solve as KB
from atomic_ops import kernel_c_recompute as KC
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


def _oracle_stages(q, k, v, w, b, g, scale):
    _, _, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 64, return_stages=True)
    return {n: torch.stack([s[n] for s in st], 2) for n in STAGES + ("Akk",)}


@pytest.mark.parametrize("dtype,K", [(F32, 64), (F32, 128), (BF16, 64), (BF16, 128)])
def test_kernels_a_b_c_alone_match_the_oracle(dtype, K):
    """Each kernel on the oracle's inputs to that kernel, against the oracle's
    outputs of it: A on q, k, b, g; B on the oracle's Akk (in the operand
    type, against the oracle's inverse of that same Akk); C on the oracle's A."""
    B, T, H = 2, 192, 2
    banner(f"gdn2 kernels A, B, C alone {dtype} K{K}")
    q, k, v, w, b, g = _inputs(B, T, H, K, dtype, 71 + K)
    ref = _oracle_stages(q, k, v, w, b, g, 0.7)
    dq, dk, dv, dw, db, dg = (t.cuda() for t in (q, k, v, w, b, g))
    tol = tol_for(dtype)
    Aqk, Akk = KA.build_chunk_scores_pallas(dq, dk, db, dg, 0.7, block=64)
    akk_in = ref["Akk"].to(dtype)
    A = KB.wy_solve_pallas(akk_in.cuda())
    A_ref = og.n2n(og.wy_inverse(akk_in.double()))
    outs = KC.recompute_wy_pallas(dq, dk, dv, dw, db, dg, ref["A"].to(dtype).cuda())
    torch.cuda.synchronize()
    checks = [("Aqk", Aqk, ref["Aqk"]), ("Akk", Akk, ref["Akk"]), ("A", A, A_ref)]
    checks += [(n, t, ref[n]) for n, t in zip(STAGES[2:], outs)]
    for name, t, r in checks:
        e = rel_err(t, r)
        print(f"  {name}: rel_err {e:.2e}")
        assert t.shape == r.shape and t.dtype == (F32 if name == "gc_last" else dtype) and e < tol, name
    # the strictly upper part of the scores is zero, the diagonal of Akk too
    assert torch.count_nonzero(torch.triu(Aqk.float(), 1)).item() == 0
    assert torch.count_nonzero(torch.triu(Akk.float(), 0)).item() == 0
    # (I + Akk) A = I for the solve's own input
    eye = torch.eye(64, dtype=torch.float64)
    resid = (eye + akk_in.double()) @ A.cpu().double() - eye
    print(f"  max |(I + Akk) A - I| = {resid.abs().max().item():.2e}")
    assert resid.abs().max().item() < (1e-5 if dtype == F32 else 5e-3)


def test_kernels_a_b_c_chained_equal_the_one_pass_build_in_fp32():
    """fp32: Akk leaves kernel A in fp32, so A -> B -> C gives the one-pass
    build's arrays bit for bit (kernel C's wider product only adds zeros)."""
    B, T, H, K = 2, 256, 2, 128
    banner("gdn2 kernels A -> B -> C vs the one-pass build (fp32)")
    q, k, v, w, b, g = (t.cuda() for t in _inputs(B, T, H, K, F32, 81))
    one = KD.build_chunk_wy(q, k, v, w, b, g, 0.9)
    Aqk, Akk = KA.build_chunk_scores_pallas(q, k, b, g, 0.9, block=64)
    A = KB.wy_solve_pallas(Akk)
    wp, u, kg, qg, gl = KC.recompute_wy_pallas(q, k, v, w, b, g, A)
    torch.cuda.synchronize()
    for name, x, y in zip(STAGES, (Aqk, A, wp, u, kg, qg, gl), one):
        assert torch.equal(x, y), name


def test_kernel_c_clips_like_the_reference():
    """Kernel C alone clips w_pseudo and u to +-1e4 (kernel_c_recompute.py:74-78):
    a large A drives them past it."""
    B, T, H, K = 1, 64, 1, 64
    banner("gdn2 kernel C clip")
    q, k, v, w, b, g = (t.cuda() for t in _inputs(B, T, H, K, F32, 91))
    A = torch.full((B, H, 1, 64, 64), 1e6, device="cuda")
    wp, u, kg, qg, gl = KC.recompute_wy_pallas(q, k, v, 10 * torch.ones_like(w), b, g, A)
    torch.cuda.synchronize()
    assert wp.abs().max().item() <= 1e4 and u.abs().max().item() == 1e4


def test_stage_entries_reject_other_chunks():
    banner("gdn2 stage chunk check")
    q, k, v, w, b, g = (t.cuda() for t in _inputs(1, 256, 2, 64, F32, 3))
    with pytest.raises(_lib.AtomicError):
        KD.gdn2_inter_chunk_combine(*(torch.zeros(1, 2, 2, 128, n, device="cuda") for n in (128, 64, 64, 64, 64)),
                                    torch.zeros(1, 2, 2, 64, device="cuda"), 1.0)
    with pytest.raises(ValueError):
        KB.wy_solve_pallas(torch.zeros(1, 2, 2, 128, 128, device="cuda"))


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_combine_with_state_and_residuals(dtype):
    """gdn2_inter_chunk_combine_with_state / gdn2_pallas_forward_with_residuals
    (kernel_d_pipeline.py:127,199): o, h_final equal to the plain combine and
    the whole forward; h_pre_all and v_new_all against the oracle's scan of
    the same stages, in the reference's [NT, B, H, ., .] order."""
    B, T, H, K = 2, 192, 2, 128
    banner(f"gdn2 combine with state {dtype}")
    q, k, v, w, b, g = _inputs(B, T, H, K, dtype, 95)
    h0 = 0.4 * torch.randn(B, H, K, K, generator=torch.Generator().manual_seed(96))
    dq, dk, dv, dw, db, dg = (t.cuda() for t in (q, k, v, w, b, g))
    o, hf, res = KD.gdn2_pallas_forward_with_residuals(dq, dk, dv, dw, db, dg, 0.6, h0=h0.cuda(), block=64)
    o_w, h_w, _ = G.forward(dq, dk, dv, dw, db, dg, 0.6, h0=h0.cuda())
    torch.cuda.synchronize()
    tol = tol_for(dtype)
    assert rel_err(o, o_w) < tol and rel_err(hf, h_w) < tol
    # the states of the scan against the oracle on the device's own stages
    st = [res[n].float().cpu() for n in ("Aqk", "w_pseudo", "u", "kg", "qg", "gc_last")]
    h = h0.double()
    NT = T // 64
    for n in range(NT):
        Aqk_c, wp_c, u_c, kg_c, qg_c, gl_c = (t[:, :, n].double() for t in st)
        v_new = u_c - wp_c @ h
        e_h, e_v = rel_err(res["h_pre_all"][n], h), rel_err(res["v_new_all"][n], v_new)
        print(f"  chunk {n}: h_pre {e_h:.2e} v_new {e_v:.2e}")
        assert res["h_pre_all"].shape == (NT, B, H, K, K) and e_h < tol and e_v < tol
        h = og.sanitize(h * torch.exp(gl_c)[..., None] + kg_c.transpose(-1, -2) @ v_new)
    assert set(res) == {"Aqk", "Akk", "A", "h_pre_all", "v_new_all", "w_pseudo", "u", "kg", "qg", "gc_last"}
