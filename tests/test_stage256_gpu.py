"""Stage-level entries at the reference's 256-row block, on the GPU.

GDN2 kernels A, B, C, D at BT = 256 with float32 arrays
(build_chunk_scores_pallas, wy_solve_pallas, recompute_wy_pallas,
gdn2_inter_chunk_combine(_with_state): kernel_a_scores.py:26-98,
kernel_b_solve.py:66-171, kernel_c_recompute.py:48-123,
kernel_d_pipeline.py:94-158) and the Mamba2 stages M2, M3 (two 128-row
sub-blocks), M4 at chunk_size 256 (kernel_mamba2_a_decay.py:53-66,
kernel_mamba2_b_intra.py:61-168, kernel_mamba2_c_interchunk.py:38-87).
Each kernel runs on the oracle's inputs to it and is compared with the
oracle's restatement of that kernel; the chained stages are compared with
the composed oracle stages and with the chunked reference at chunk 256.
Every stage computes in float32 from the (bf16-rounded) inputs, as the
reference does after its upcast, so the float32 tolerance applies to both
input dtypes.
"""
import pytest
import torch

from _util import TOL_BF16, TOL_F32, banner, rel_err
from atomic_ops import inputs
from atomic_ops import kernel_a_scores as KA
from atomic_ops import kernel_b_solve as KB
from atomic_ops import kernel_c_recompute as KC
from atomic_ops import kernel_d_pipeline as KD
from atomic_ops import kernel_mamba2_a_decay as MA
from atomic_ops import kernel_mamba2_b_intra as MB
from atomic_ops import kernel_mamba2_c_interchunk as MC
from oracle import gdn2 as og
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
GIN = ("q", "k", "v", "w", "b", "g")


def _check(name, got, ref, tol=TOL_F32):
    e = rel_err(got, ref)
    print(f"  {name}: rel_err {e:.2e}", flush=True)
    assert tuple(got.shape) == tuple(ref.shape) and got.dtype == F32 and e < tol, (name, e)


@pytest.mark.parametrize("dtype,K", [(F32, 128), (BF16, 128), (F32, 64), (BF16, 64)])
def test_gdn2_block_kernels_match_the_oracle(dtype, K):
    B, T, H, scale = 2, 512, 2, 0.8
    banner(f"gdn2 stage kernels at BT 256 {dtype} K{K}")
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=101 + K, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in GIN)
    dev = [t.cuda() for t in (q, k, v, w, b, g)]
    Aqk_r, Akk_r = og.chunk_scores(q, k, b, g, scale)
    A_r = og.wy_solve_blocked(Akk_r.float().double())
    wp_r, u_r, kg_r, qg_r, gl_r = og.recompute_wy(q, k, v, w, b, g, A_r.float().double())
    Aqk, Akk = KA.build_chunk_scores_pallas(dev[0], dev[1], dev[4], dev[5], scale)
    A = KB.wy_solve_pallas(Akk_r.float().cuda())
    outs = KC.recompute_wy_pallas(*dev, A_r.float().cuda())
    torch.cuda.synchronize()
    _check("Aqk", Aqk, Aqk_r)
    _check("Akk", Akk, Akk_r)
    _check("A", A, A_r)
    for name, x, r in zip(("w_pseudo", "u", "kg", "qg", "gc_last"), outs, (wp_r, u_r, kg_r, qg_r, gl_r)):
        _check(name, x, r)
    assert torch.count_nonzero(torch.triu(Aqk, 1)).item() == 0
    assert torch.count_nonzero(torch.triu(Akk, 0)).item() == 0
    assert torch.count_nonzero(A[..., :128, 128:]).item() == 0
    eye = torch.eye(256, dtype=torch.float64)
    resid = ((eye + Akk_r.float().double()) @ A.cpu().double() - eye).abs().max().item()
    print(f"  max |(I + Akk) A - I| = {resid:.2e}")
    assert resid < 1e-4


def test_gdn2_block_solve_sanitises_like_the_reference():
    """A near-singular Akk: the entries past +-1e4 are clipped at the same
    block products as in the reference (kernel_b_solve.py:81,104,113-115,
    141,143)."""
    banner("gdn2 BT 256 solve with the clips firing")
    # -2 on the subdiagonal: (I + Akk)^-1 has entries 2^(i-j), past 1e4 from
    # 14 rows below the diagonal on; every term is positive, so the clipped
    # results do not depend on the summation order
    Akk = torch.zeros(1, 1, 2, 256, 256)
    idx = torch.arange(1, 256)
    Akk[..., idx, idx - 1] = -2.0
    A_r = og.wy_solve_blocked(Akk.double())
    assert A_r.abs().max().item() == 1e4
    A = KB.wy_solve_pallas(Akk.cuda())
    torch.cuda.synchronize()
    assert torch.isfinite(A).all()
    _check("A (clipped)", A, A_r)


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_gdn2_block_combine_matches_the_oracle(dtype):
    """Kernel D at 256-row blocks on the oracle's arrays (h0 with NaN and
    3e4, sanitised first), and the states of its scan."""
    B, T, H, K = 1, 768, 2, 128
    banner(f"gdn2 BT 256 combine {dtype}")
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=105, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in GIN)
    Aqk_r, Akk_r = og.chunk_scores(q, k, b, g, 0.6)
    A_r = og.wy_solve_blocked(Akk_r)
    arr = [Aqk_r] + list(og.recompute_wy(q, k, v, w, b, g, A_r))
    arr = [t.float().double() for t in arr]
    h0 = 0.4 * torch.randn(B, H, K, K, generator=torch.Generator().manual_seed(106))
    h0[0, 0, 0, 0], h0[0, 1, 2, 3] = float("nan"), 3e4
    o_r, h_r = og.gdn2_inter_chunk_combine(*arr, 0.6, h0=h0)
    dev = [t.float().cuda() for t in arr]
    o, hf = KD.gdn2_inter_chunk_combine(*dev, 0.6, h0=h0.cuda())
    o2, hf2, h_pre, v_new = KD.gdn2_inter_chunk_combine_with_state(*dev, 0.6, h0=h0.cuda())
    torch.cuda.synchronize()
    _check("o", o, o_r)
    _check("h_final", hf, h_r)
    assert torch.equal(o, o2) and torch.equal(hf, hf2)
    assert h_pre.shape == (3, B, H, K, K) and v_new.shape == (3, B, H, 256, K)
    h = og.sanitize(h0.double())
    for n in range(3):
        vn = arr[2][:, :, n] - arr[1][:, :, n] @ h
        _check(f"h_pre[{n}]", h_pre[n], h)
        _check(f"v_new[{n}]", v_new[n], vn)
        h = og.sanitize(h * torch.exp(arr[5][:, :, n])[..., None] + arr[3][:, :, n].transpose(-1, -2) @ vn)


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_gdn2_block_stages_chained(dtype):
    """A -> B -> C -> D at 256 rows on the GPU against the oracle's stages
    composed; in float32, also against the chunked reference at chunk 256;
    and the staged forward with residuals against the whole-path forward."""
    from atomic_ops import gdn2 as G
    B, T, H, K = 2, 512, 2, 128
    banner(f"gdn2 BT 256 chained stages {dtype}")
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=107, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in GIN)
    dev = [t.cuda() for t in (q, k, v, w, b, g)]
    Aqk, Akk = KA.build_chunk_scores_pallas(dev[0], dev[1], dev[4], dev[5], 1.0)
    A = KB.wy_solve_pallas(Akk)
    wp, u, kg, qg, gl = KC.recompute_wy_pallas(*dev, A)
    o, hf = KD.gdn2_inter_chunk_combine(Aqk, wp, u, kg, qg, gl, 1.0)
    o_s, hf_s, res = KD.gdn2_pallas_forward_with_residuals(*dev, 1.0)
    o_w, h_w, _ = G.forward(*dev, 1.0)
    torch.cuda.synchronize()
    Aqk_r, Akk_r = og.chunk_scores(q, k, b, g, 1.0)
    A_r = og.wy_solve_blocked(Akk_r)
    arr = og.recompute_wy(q, k, v, w, b, g, A_r)
    o_r, h_r = og.gdn2_inter_chunk_combine(Aqk_r, *arr, 1.0)
    _check("o", o, o_r)
    _check("h_final", hf, h_r)
    if dtype == F32:
        oc, hc = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 256)
        _check("o vs chunked reference", o.permute(0, 2, 3, 1, 4).reshape(B, T, H, K), oc)
        _check("h_final vs chunked reference", hf, hc)
    assert torch.equal(o_s, o.permute(0, 2, 3, 1, 4).reshape(B, T, H, K)) and torch.equal(hf_s, hf)
    assert res["A"].shape == (B, H, 2, 256, 256) and res["h_pre_all"].shape == (2, B, H, K, K)
    # the whole path runs 64-row chunks: equal up to the exp(-20) floors and rounding
    _check("staged vs whole path", o_s, o_w, TOL_BF16)


@pytest.mark.parametrize("B,T,H,P,N", [
    (2, 512, 2, 64, 128),
    (1, 512, 2, 128, 64),
    (1, 768, 2, 128, 128),
    (1, 512, 2, 192, 128),    # the model's headdim at the model's chunk
])
def test_mamba2_chunk256_stages_match_the_oracle(B, T, H, P, N):
    banner(f"mamba2 stages at chunk 256 B{B} T{T} H{H} P{P} N{N}")
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=T + P + N)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    s0 = 0.3 * torch.randn(B, H, P, N, generator=torch.Generator().manual_seed(9))
    s0[0, 0, 0, 0], s0[0, -1, 1, 1] = float("nan"), 3e4        # sanitised by M4
    cum_r = om.build_chunk_cumdecay(dt, A, 256)
    yd_r, se_r = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_r, 256)
    y_r, sf_r = om.mamba2_inter_chunk_combine(yd_r, se_r, cum_r, Cm, 256, state0=s0)
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    cum = MA.build_chunk_cumdecay_pallas(g[0], g[4], 256)
    yd, se = MB.intra_chunk_ssd_pallas(g[0], g[1], g[2], g[3], cum_r.float().cuda(), 256)
    y, sf = MC.mamba2_inter_chunk_combine(yd_r.float().cuda(), se_r.float().cuda(), cum_r.float().cuda(), g[3], 256,
                                          state0=s0.cuda())
    ys, sfs = MC.mamba2_pallas_forward(*g, 256, state0=s0.cuda())
    torch.cuda.synchronize()
    _check("cumdecay", cum, cum_r)
    _check("y_diag", yd, yd_r)
    _check("state_end", se, se_r)
    _check("y", y, y_r)
    _check("state_final", sf, sf_r)
    _check("staged y", ys, y_r)
    _check("staged state_final", sfs, sf_r)


def test_mamba2_chunk256_sub_blocks_are_sanitised_apart():
    """M3 at chunk 256 adds the second 128-row half's part from the first
    half's sources as its own sanitised sum (kernel_mamba2_b_intra.py:88-108):
    with dBx large enough that this cross part passes +-1e4, y_diag of the
    second half equals the oracle's sub-block form, not one sum over all
    sources."""
    B, T, H, P, N = 1, 256, 1, 64, 64
    banner("mamba2 chunk 256 sub-block sanitise")
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=11)
    d["x"] = (d["x"].float() * 3e3).to(BF16)
    d["Bm"] = (d["Bm"].float() * 8).to(BF16)
    d["Cm"] = (d["Cm"].float() * 8).to(BF16)
    d["A"] = d["A"] * 0.01
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    cum_r = om.build_chunk_cumdecay(dt, A, 256)
    yd_r, _ = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_r, 256)
    assert yd_r.abs().max().item() == 1e4, "the clips must bind"
    yd, _ = MB.intra_chunk_ssd_pallas(*(t.cuda() for t in (dt, x, Bm, Cm)), cum_r.float().cuda(), 256)
    torch.cuda.synchronize()
    _check("y_diag", yd, yd_r)
