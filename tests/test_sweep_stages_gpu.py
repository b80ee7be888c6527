"""Seeded random shapes of the stage-level entries on the GPU against the
float64 oracle: the GDN2 stage chain at the reference's 256-row block
(kernels A, B, C, D with state, then B2, B1, B3, B4, B5, composed as
_gdn2_core_bwd, kernel_trainable_B6.py:97-181) against the oracle's staged
backward; the Mamba2 MB1 + MB3 scan (kernel_mamba2_bwd_b1_state.py:132-254)
against its restatement and, with MB4, against MB0; the Mamba2 staged
forward (M2 -> M3 -> M4, kernel_mamba2_c_interchunk.py:50-53) against the
oracle's stages.  Batch 1-3, 1-3 blocks or chunks, 1-4 heads, chunks 64 /
128 / 256, every Mamba2 head size.  The stage entries compute in float32,
except the Mamba2 forward stages on bf16 operands, which run the bf16
kernels (2e-2)."""
import random

import pytest
import torch

from _util import TOL_F32, banner, rel_err, tol_for
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
from atomic_ops import kernel_mamba2_bwd_b1_state as MB1
from atomic_ops import kernel_mamba2_c_interchunk as MC
from atomic_ops import mamba2_bwd_a_dA_reference as MB4
from oracle import gdn2 as og
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
BT = 256


def _fin(t):
    return torch.nan_to_num(torch.clamp(t, -1e4, 1e4), nan=0.0)


def _dev(t, dt=F32):
    return t.to(dt).contiguous().cuda()


def _check(errs, tol):
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < tol, (k, v, tol)


def _cases(seed, n):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        if i % 3 == 0:
            # kernel B4 takes K = 128 only, as the reference's does (kernel_bwd_b4_intra.py:137)
            out.append(("gdn2_chain", (rng.choice([1, 2, 3]), BT * rng.choice([1, 2, 3]), rng.choice([1, 2, 3]), 128,
                                       rng.choice([F32, BF16]), rng.choice([1.0, 0.8, 128 ** -0.5]),
                                       rng.randrange(1000))))
            continue
        b = rng.choice([1, 2, 3]); C = rng.choice([64, 128, 256]); l = C * rng.choice([1, 2, 3])
        h = rng.choice([1, 2, 3, 4]); P = rng.choice([64, 128, 192]); N = 128 if P == 192 else rng.choice([64, 128])
        kind = "mamba2_scan" if i % 3 == 1 else "mamba2_fwd"
        out.append((kind, (b, l, h, P, N, C, rng.choice([F32, BF16]), rng.randrange(1000))))
    return out


CASES = _cases(3, 45)


def _name(c):
    kind, a = c
    return kind + "-" + "-".join(str(v).replace("torch.", "") if not isinstance(v, float) else f"{v:.3f}" for v in a)


def _gdn2_chain(B, T, H, K, dtype, s, seed):
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype)
    q, k, v, w, b, g = (d[n] for n in ("q", "k", "v", "w", "b", "g"))
    gen = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(B, T, H, K, generator=gen).to(dtype)
    dhf = 0.3 * torch.randn(B, H, K, K, generator=gen)
    h0 = 0.3 * torch.randn(B, H, K, K, generator=gen)
    ref = og.gdn2_backward_staged(q, k, v, w, b, g, s, do, dh_final=dhf, h0=h0)
    qd, kd, vd, wd, bd = (_dev(t, dtype) for t in (q, k, v, w, b))
    gd, dod = _dev(g), _dev(do, dtype)
    Aqk, Akk = KA.build_chunk_scores_pallas(qd, kd, bd, gd, s)
    A = KB.wy_solve_pallas(Akk)
    wp, u, kg, qg, gcl = KC.recompute_wy_pallas(qd, kd, vd, wd, bd, gd, A)
    _, _, h_pre, v_new = KD.gdn2_inter_chunk_combine_with_state(Aqk, wp, u, kg, qg, gcl, s, h0=_dev(h0))
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
    got = (_fin(unblk(b3["dq"] + dq4)), _fin(unblk(b3["dk"] + dk4)), _fin(unblk(b3["dv_raw"])),
           _fin(unblk(b3["dw"])), _fin(unblk(b3["db"] + db4)), _fin(unblk(dg)), _fin(dh0))
    torch.cuda.synchronize()
    _check({n: rel_err(x, r) for n, x, r in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), got, ref)}, TOL_F32)


def _mamba2_scan(b, l, h, P, N, C, dyt, seed):
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=seed, dO=True)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    gen = torch.Generator().manual_seed(seed + 1)
    dy = torch.randn(b, l, h, P, generator=gen).to(dyt)
    dsf = 0.3 * torch.randn(b, h, P, N, generator=gen)
    s0 = 0.3 * torch.randn(b, h, P, N, generator=gen)
    ref = om.mamba2_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    got = MB1.mamba2_bwd_scan(dt.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), x.cuda(), C, dy.cuda(), dsf.cuda(),
                              state0=s0.cuda())
    dtp = MB4.reshape_dt_to_pallas(dt, C)
    ddt2, dA = MB4.mamba2_dA_backward(dtp.cuda(), A.cuda(), got[5], C)
    comp = (_fin(got[0] + MB4.unreshape_dt_from_pallas(ddt2)), _fin(got[1]), _fin(got[2]), _fin(got[3]), _fin(dA),
            _fin(got[4]))
    torch.cuda.synchronize()
    mb0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    errs = {"scan " + n: rel_err(g_, r)
            for n, g_, r in zip(("ddt", "dB", "dC", "dx", "dstate0", "dcumdecay"), got, ref)}
    errs.update({"vs MB0 " + n: rel_err(g_, om.final_sanitize(r))
                 for n, g_, r in zip(("ddt", "dB", "dC", "dx", "dA", "dstate0"), comp, mb0)})
    _check(errs, TOL_F32)


def _mamba2_fwd(b, l, h, P, N, C, dtype, seed):
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=seed, dtype=dtype)
    dt, x, Bm, Cm, A = (d[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    s0 = 0.3 * torch.randn(b, h, P, N, generator=torch.Generator().manual_seed(seed + 3))
    ys, sfs = MC.mamba2_pallas_forward(*[t.cuda() for t in (dt, x, Bm, Cm, A)], C, state0=s0.cuda())
    torch.cuda.synchronize()
    cum = om.build_chunk_cumdecay(dt, A, C)
    yd, se = om.intra_chunk_ssd(dt, x, Bm, Cm, cum, C)
    y_r, sf_r = om.mamba2_inter_chunk_combine(yd, se, cum, Cm, C, state0=s0)
    _check({"y": rel_err(ys, y_r), "state_final": rel_err(sfs, sf_r)}, tol_for(dtype))


@pytest.mark.parametrize("case", CASES, ids=[_name(c) for c in CASES])
def test_random_shapes_of_the_stage_entries(case):
    kind, args = case
    banner(_name(case))
    {"gdn2_chain": _gdn2_chain, "mamba2_scan": _mamba2_scan, "mamba2_fwd": _mamba2_fwd}[kind](*args)
