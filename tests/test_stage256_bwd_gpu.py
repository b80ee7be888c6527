"""Backward stage entries at the reference's 256-row block, on the GPU.

GDN2 kernels B2, B1, B3, B4, B5 (dav_backward_pallas, gdn2_dhu_backward,
wy_dqkg_backward_pallas, intra_backward_pallas, reverse_cumsum_bwd:
kernel_bwd_b2_dav.py:17-51, kernel_bwd_b1_dhu.py:14-44,
kernel_bwd_b3_wy_dqkg.py:33-148, kernel_bwd_b4_intra.py:57-165,
kernel_bwd_b5_reverse_cumsum.py:17-24).  Each entry runs on the oracle's
inputs to it (rounded to float32, as the entries take them) and is compared
with the oracle's restatement of that kernel; the whole chain of stage
entries, forward kernels A-D included, is compared with the oracle's staged
backward (pinned against autodiff of the chunked reference).  Every stage
computes in float32, so the float32 tolerance applies to both input dtypes.
"""
import pytest
import torch

from _util import TOL_F32, banner, rel_err
from atomic_ops import inputs
from atomic_ops import kernel_a_scores as KA
from atomic_ops import kernel_b_solve as KB
from atomic_ops import kernel_bwd_b1_dhu as B1
from atomic_ops import kernel_bwd_b2_dav as B2
from atomic_ops import kernel_bwd_b3_wy_dqkg as B3
from atomic_ops import kernel_bwd_b4_intra as B4
from atomic_ops import kernel_bwd_b5_reverse_cumsum as B5
from atomic_ops import kernel_c_recompute as KC
from atomic_ops import kernel_d_pipeline as KD
from oracle import gdn2 as og

pytestmark = pytest.mark.gpu

F32, BF16, F64 = torch.float32, torch.bfloat16, torch.float64
BT = 256


def _check(name, got, ref, tol=TOL_F32):
    e = rel_err(got, ref)
    print(f"  {name}: rel_err {e:.2e}", flush=True)
    assert tuple(got.shape) == tuple(ref.shape) and got.dtype == F32 and e < tol, (name, e)


def _r(t):
    """The float32 rounding the entries see, back in float64 for the oracle."""
    return t.float().double()


def _positive_gates(g):
    """Head 0's gates made positive (0.02 |g|, so gc grows along a block and
    the pair decays exceed 1): the stage kernels' clips then act where the
    model's gates (g <= 0) never take them."""
    g = g.clone()
    g[:, :, 0] = 0.02 * g[:, :, 0].abs()
    return g


def _case(B, T, H, K, dtype, seed, scale=0.8, positive=False):
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in ("q", "k", "v", "w", "b", "g"))
    if positive:
        g = _positive_gates(g)
    gen = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(B, T, H, K, generator=gen).to(dtype)
    dht = 0.3 * torch.randn(B, H, K, K, generator=gen)
    Aqk, Akk = og.chunk_scores(q, k, b, g, scale)
    A = og.wy_solve_blocked(_r(Akk))
    wp, u, kg, qg, gcl = og.recompute_wy(q, k, v, w, b, g, _r(A))
    _, _, h_pre, v_new = og.gdn2_inter_chunk_combine(_r(Aqk), _r(wp), _r(u), _r(kg), _r(qg), _r(gcl), scale,
                                                     return_state=True)
    blk = lambda t: og._blocks(t.double(), BT)
    return dict(q=q, k=k, v=v, w=w, b=b, g=g, do=do, dht=dht, scale=scale, Aqk=Aqk, Akk=Akk, A=A, wp=wp,
                u=u, kg=kg, qg=qg, gcl=gcl, h_pre=h_pre, v_new=v_new, blk=blk,
                gc=torch.cumsum(blk(g), dim=-2))


def _dev(t, dtype=F32):
    return t.to(dtype).contiguous().cuda()


@pytest.mark.parametrize("dtype,K,positive", [(F32, 128, False), (BF16, 128, False), (F32, 64, False),
                                              (BF16, 64, False), (F32, 128, True)])
def test_gdn2_backward_block_kernels_match_the_oracle(dtype, K, positive):
    B, T, H = 1, 512, 2
    banner(f"gdn2 backward stage kernels at BT 256 {dtype} K{K}{' positive gates' if positive else ''}")
    c = _case(B, T, H, K, dtype, seed=301 + K, positive=positive)
    s = c["scale"]
    blk = c["blk"]
    do_b = blk(c["do"])
    # B2
    dAqk_r, dvp_r = og.dav_backward(_r(c["Aqk"]), _r(c["v_new"]), do_b)
    dAqk, dvp = B2.dav_backward_pallas(_dev(c["Aqk"]), _dev(c["v_new"]), _dev(do_b, dtype))
    torch.cuda.synchronize()
    _check("B2 dAqk", dAqk, dAqk_r)
    _check("B2 dv_new", dvp, dvp_r)
    assert torch.count_nonzero(torch.triu(dAqk, 1)).item() == 0
    # B1
    dh_all_r, dh0_r, dv_all_r = og.dhu_backward(do_b, _r(dvp_r), _r(c["wp"]), _r(c["qg"]), _r(c["kg"]),
                                                _r(c["gcl"]), s, dht=_r(c["dht"]))
    dh_all, dh0, dv_all = B1.gdn2_dhu_backward(_dev(do_b, dtype), _dev(dvp_r), _dev(c["wp"]), _dev(c["qg"]),
                                               _dev(c["kg"]), _dev(c["gcl"]), s, dht=_dev(c["dht"]))
    torch.cuda.synchronize()
    _check("B1 dh_all", dh_all, dh_all_r)
    _check("B1 dh0", dh0, dh0_r)
    _check("B1 dv_all", dv_all, dv_all_r)
    # B3
    dh_next_r = torch.cat([dh_all_r[:, :, 1:], _r(c["dht"])[:, :, None]], dim=2)
    qb, kb, bb, wb, vb = (blk(c[n]) for n in ("q", "k", "b", "w", "v"))
    b3_r = og.wy_dqkg_backward(qb, kb, bb, wb, vb, _r(c["gc"]), _r(c["A"]), c["Akk"], _r(c["h_pre"]),
                               _r(c["v_new"]), do_b, _r(dv_all_r), _r(dh_next_r), s)
    b3 = B3.wy_dqkg_backward_pallas(*(_dev(t, dtype) for t in (qb, kb, bb, wb, vb)), _dev(c["gc"]), _dev(c["A"]),
                                    _dev(c["Akk"]), _dev(c["h_pre"]), _dev(c["v_new"]), _dev(do_b, dtype),
                                    _dev(dv_all_r), _dev(dh_next_r), s)
    torch.cuda.synchronize()
    for n in ("dq", "dk", "db", "dw", "dv_raw", "dgc", "dAkk"):
        _check(f"B3 {n}", b3[n], b3_r[n])
    assert torch.count_nonzero(torch.triu(b3["dAkk"], 0)).item() == 0
    # B4 (the reference takes K = 128 only)
    dgc4_r = None
    if K == 128:
        outs_r = og.intra_backward(_r(dAqk_r), _r(b3_r["dAkk"]), c["q"], c["k"], c["b"], c["g"], s)
        outs = B4.intra_backward_pallas(_dev(dAqk_r), _dev(b3_r["dAkk"]), _dev(c["q"], dtype), _dev(c["k"], dtype),
                                        _dev(c["b"], dtype), _dev(c["g"]), s)
        torch.cuda.synchronize()
        for n, x, r in zip(("dq", "dk", "db", "dgc"), outs, outs_r):
            _check(f"B4 {n}", x, r)
        dgc4_r = outs_r[3]
    else:
        with pytest.raises(ValueError):
            B4.intra_backward_pallas(_dev(dAqk_r), _dev(b3_r["dAkk"]), _dev(c["q"], dtype), _dev(c["k"], dtype),
                                     _dev(c["b"], dtype), _dev(c["g"]), s)
    # B5
    dgc_tot = b3_r["dgc"] + (dgc4_r if dgc4_r is not None else 0.0)
    dg = B5.reverse_cumsum_bwd(_dev(dgc_tot), BT)
    torch.cuda.synchronize()
    _check("B5 dg", dg, og.reverse_cumsum_bwd(_r(dgc_tot), BT))


def test_gdn2_backward_stages_sanitise_like_the_reference():
    """dht with NaN / +-inf / 3e4 is sanitised before the scan
    (kernel_bwd_b1_dhu.py:16-18); B4 with partial sums past +-1e4 clips after
    every accumulation (kernel_bwd_b4_intra.py:113-121)."""
    B, T, H, K = 1, 512, 2, 128
    banner("gdn2 backward stages: sanitise points")
    c = _case(B, T, H, K, F32, seed=77)
    s = c["scale"]
    do_b = c["blk"](c["do"])
    dht = c["dht"].clone()
    dht[0, 0, 0, :4] = torch.tensor([float("nan"), float("inf"), -float("inf"), 3e4])
    dvp_r = og.dav_backward(_r(c["Aqk"]), _r(c["v_new"]), do_b)[1]
    ref = og.dhu_backward(do_b, _r(dvp_r), _r(c["wp"]), _r(c["qg"]), _r(c["kg"]), _r(c["gcl"]), s, dht=dht.double())
    got = B1.gdn2_dhu_backward(_dev(do_b), _dev(dvp_r), _dev(c["wp"]), _dev(c["qg"]), _dev(c["kg"]), _dev(c["gcl"]),
                               s, dht=_dev(dht))
    torch.cuda.synchronize()
    for n, x, r in zip(("dh_all", "dh0", "dv_all"), got, ref):
        assert torch.isfinite(x).all(), n
        _check(f"B1 {n} (non-finite dht)", x, r)
    # sub-block pair (1, 0) far past the clip with every term positive (q, k
    # taken positive, no decay: no cancellation, so float32 and float64 agree
    # on each clipped value), (1, 1) moderate: rows 128..255 of dq are
    # clip(clip(huge) + moderate), inside +-1e4 where the moderate part is
    # negative (a clip at the end only would leave them at 1e4)
    gen = torch.Generator().manual_seed(5)
    dAqk = torch.randn(B, H, 2, BT, BT, generator=gen)
    dAqk[..., 128:, :128] = 1e8 * dAqk[..., 128:, :128].abs()
    dAkk = torch.randn(B, H, 2, BT, BT, generator=gen)
    qp, kp, g0 = c["q"].abs(), c["k"].abs(), torch.zeros_like(c["g"])
    ref4 = og.intra_backward(dAqk.double(), dAkk.double(), qp, kp, c["b"], g0, s)
    got4 = B4.intra_backward_pallas(_dev(dAqk), _dev(dAkk), _dev(qp), _dev(kp), _dev(c["b"]), _dev(g0), s)
    torch.cuda.synchronize()
    for n, x, r in zip(("dq", "dk", "db", "dgc"), got4, ref4):
        assert torch.isfinite(x).all() and x.abs().max().item() <= 1e4, n
        _check(f"B4 {n} (clipped partial sums)", x, r)
    lower = got4[0][..., 128:, :].abs()
    inside = ((lower > 9e3) & (lower < 1e4 - 1e-2)).sum().item()
    print(f"  dq rows 128..255 between 9e3 and 1e4: {inside}", flush=True)
    assert inside > 0


@pytest.mark.parametrize("dtype,positive", [(F32, False), (BF16, False), (F32, True)])
def test_gdn2_backward_stage_chain_matches_the_staged_oracle(dtype, positive):
    """Kernels A, B, C, D-with-state, then B2, B1, B3, B4, B5 through the
    stage entries, composed as _gdn2_core_bwd (kernel_trainable_B6.py:97-181);
    also with head 0's gates positive."""
    B, T, H, K = 1, 512, 2, 128
    banner(f"gdn2 backward stage chain {dtype}{' positive gates' if positive else ''}")
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=55, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in ("q", "k", "v", "w", "b", "g"))
    if positive:
        g = _positive_gates(g)
    gen = torch.Generator().manual_seed(56)
    do = torch.randn(B, T, H, K, generator=gen).to(dtype)
    dhf = 0.3 * torch.randn(B, H, K, K, generator=gen)
    h0 = 0.3 * torch.randn(B, H, K, K, generator=gen)
    s = 0.8
    ref = og.gdn2_backward_staged(q, k, v, w, b, g, s, do, dh_final=dhf, h0=h0)
    dq_, dk_, dv_, dw_, db_, dg_, dh0_ = ref
    qd, kd, vd, wd, bd = (_dev(t, dtype) for t in (q, k, v, w, b))
    gd, dod = _dev(g), _dev(do, dtype)
    Aqk, Akk = KA.build_chunk_scores_pallas(qd, kd, bd, gd, s)
    A = KB.wy_solve_pallas(Akk)
    wp, u, kg, qg, gcl = KC.recompute_wy_pallas(qd, kd, vd, wd, bd, gd, A)
    _, _, h_pre, v_new = KD.gdn2_inter_chunk_combine_with_state(Aqk, wp, u, kg, qg, gcl, s, h0=_dev(h0))
    # scan order [NT, B, H, ...] -> [B, H, NT, ...] (kernel_trainable_B6.py:109-110)
    h_pre, v_new = h_pre.movedim(0, 2).contiguous(), v_new.movedim(0, 2).contiguous()
    blk = lambda t: t.reshape(B, T // BT, BT, H, K).permute(0, 3, 1, 2, 4).contiguous()
    unblk = lambda t: t.permute(0, 2, 3, 1, 4).reshape(B, T, H, K)
    gc = torch.cumsum(blk(gd), dim=-2)
    dAqk, dvp = B2.dav_backward_pallas(Aqk, v_new, blk(dod))
    dh_all, dh0, dv_all = B1.gdn2_dhu_backward(blk(dod), dvp, wp, qg, kg, gcl, s, dht=_dev(dhf))
    dh_next = torch.cat([dh_all[:, :, 1:], _dev(dhf)[:, :, None]], dim=2)
    b3 = B3.wy_dqkg_backward_pallas(blk(qd), blk(kd), blk(bd), blk(wd), blk(vd), gc, A, Akk, h_pre, v_new, blk(dod),
                                    dv_all, dh_next, s)
    dq4, dk4, db4, dgc4 = B4.intra_backward_pallas(dAqk, b3["dAkk"], qd, kd, bd, gd, s)
    dg = B5.reverse_cumsum_bwd(b3["dgc"] + dgc4, BT)
    fin = lambda t: torch.nan_to_num(torch.clamp(t, -1e4, 1e4), nan=0.0)
    got = (fin(unblk(b3["dq"] + dq4)), fin(unblk(b3["dk"] + dk4)), fin(unblk(b3["dv_raw"])), fin(unblk(b3["dw"])),
           fin(unblk(b3["db"] + db4)), fin(unblk(dg)), fin(dh0))
    torch.cuda.synchronize()
    for n, x, r in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), got, ref):
        _check(f"chain {n}", x, r)


# ---------------------------------------------------------------- Mamba2 MB2
from atomic_ops import kernel_mamba2_bwd_b2_intra as MB2  # noqa: E402
from oracle import mamba2 as om  # noqa: E402


@pytest.mark.parametrize("C,P,N,dy_dtype", [(256, 64, 128, BF16), (256, 128, 64, F32), (128, 64, 64, F32),
                                            (64, 128, 128, BF16)])
def test_mamba2_intra_backward_matches_the_oracle(C, P, N, dy_dtype):
    """MB2 (kernel_mamba2_bwd_b2_intra.py:32-180) against the oracle's
    restatement (itself the vector-Jacobian product of M3) on the bf16
    inputs, the oracle's cumdecay and random cotangents."""
    b, l, h = 1, 512, 2
    banner(f"mamba2 MB2 chunk {C} P{P} N{N} dy {dy_dtype}")
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=400 + C + P, device=torch.device("cpu"), dO=True)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    gen = torch.Generator().manual_seed(401 + C)
    dy = torch.randn(b, l, h, P, generator=gen).to(dy_dtype)
    dse = 0.3 * torch.randn(b, h, l // C, P, N, generator=gen)
    cum = om.build_chunk_cumdecay(dt, A, C).float()
    ref = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum.double(), dy.double(), dse.double(), C)
    got = MB2.intra_chunk_ssd_bwd_pallas(dt.cuda(), x.cuda(), Bm.cuda(), Cm.cuda(), cum.cuda(), dy.cuda(),
                                         dse.cuda(), C)
    torch.cuda.synchronize()
    for n, g_, r in zip(("ddt", "dx", "dB", "dC", "dcum"), got, ref):
        _check(f"MB2 {n}", g_, r)


def test_mamba2_intra_backward_sanitises_every_sub_block():
    """A cotangent large enough that single sub-block pair sums pass +-1e4:
    every output finite, within +-1e4 and equal to the oracle's."""
    b, l, h, P, N, C = 1, 256, 2, 64, 64, 256
    banner("mamba2 MB2 sanitise points")
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=407, device=torch.device("cpu"), dO=True)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    gen = torch.Generator().manual_seed(408)
    dy = torch.randn(b, l, h, P, generator=gen)
    dy[:, 128:] = 1e7 * dy[:, 128:].abs()
    dse = torch.randn(b, h, 1, P, N, generator=gen)
    cum = om.build_chunk_cumdecay(dt, A, C).float()
    ref = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum.double(), dy.double(), dse.double(), C)
    got = MB2.intra_chunk_ssd_bwd_pallas(dt.cuda(), x.cuda(), Bm.cuda(), Cm.cuda(), cum.cuda(), dy.cuda(),
                                         dse.cuda(), C)
    torch.cuda.synchronize()
    for n, g_, r in zip(("ddt", "dx", "dB", "dC", "dcum"), got, ref):
        assert torch.isfinite(g_).all(), n
        _check(f"MB2 {n} (large dy)", g_, r)


# ---------------------------------------------------------------- Mamba2 MB1 + MB3, MB4
from atomic_ops import kernel_mamba2_bwd_b1_state as MB1  # noqa: E402
from atomic_ops import mamba2_bwd_a_dA_reference as MB4  # noqa: E402


def _m2_full(b, l, h, P, N, seed, dy_dtype):
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=seed, device=torch.device("cpu"), dO=True)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    gen = torch.Generator().manual_seed(seed + 1)
    dy = torch.randn(b, l, h, P, generator=gen).to(dy_dtype)
    dsf = 0.3 * torch.randn(b, h, P, N, generator=gen)
    s0 = 0.3 * torch.randn(b, h, P, N, generator=gen)
    return dt, x, Bm, Cm, A, dy, dsf, s0


@pytest.mark.parametrize("C,P,N,dy_dtype", [(256, 64, 128, BF16), (128, 128, 64, F32), (64, 64, 128, F32)])
def test_mamba2_bwd_scan_and_da_match_the_oracle(C, P, N, dy_dtype):
    """MB1 + MB3 (kernel_mamba2_bwd_b1_state.py:132-254) and MB4
    (mamba2_bwd_a_dA_reference.py:60-115) against the oracle's restatements
    (composed, they equal MB0), then composed as the trainable op
    (kernel_mamba2_trainable_B6.py:83-131) against MB0 itself."""
    b, l, h = 1, 512, 2
    banner(f"mamba2 MB1+MB3, MB4 chunk {C} P{P} N{N} dy {dy_dtype}")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _m2_full(b, l, h, P, N, 500 + C + P, dy_dtype)
    ref = om.mamba2_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    got = MB1.mamba2_bwd_scan(dt.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), x.cuda(), C, dy.cuda(), dsf.cuda(),
                              state0=s0.cuda())
    torch.cuda.synchronize()
    for n, g_, r in zip(("ddt", "dB", "dC", "dx", "dstate0", "dcumdecay"), got, ref):
        _check(f"MB1+MB3 {n}", g_, r)
    dtp = MB4.reshape_dt_to_pallas(dt, C)
    ref4 = om.mamba2_dA_backward(dtp, A, ref[5], C)
    got4 = MB4.mamba2_dA_backward(dtp.cuda(), A.cuda(), ref[5].float().cuda(), C)
    torch.cuda.synchronize()
    _check("MB4 ddt_contrib2", got4[0], ref4[0])
    _check("MB4 dA", got4[1], ref4[1])
    # the trainable op's composition against MB0
    ddt2, dA = MB4.mamba2_dA_backward(dtp.cuda(), A.cuda(), got[5], C)
    fin = lambda t: torch.nan_to_num(torch.clamp(t, -1e4, 1e4), nan=0.0)
    comp = (fin(got[0] + MB4.unreshape_dt_from_pallas(ddt2)), fin(got[1]), fin(got[2]), fin(got[3]), fin(dA),
            fin(got[4]))
    mb0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    torch.cuda.synchronize()
    for n, g_, r in zip(("ddt", "dB", "dC", "dx", "dA", "dstate0"), comp, mb0):
        _check(f"composed vs MB0 {n}", g_, om.final_sanitize(r))
