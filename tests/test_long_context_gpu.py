"""Configuration 4 (B1 T32768: 512 GDN2 chunks, 256 Mamba2 chunks) on the GPU.

The fp64 oracle cannot run every head at this length in test time, so each
path is checked three ways at the full shape:
  * one head of the full-shape inputs through the oracle (forward and
    backward), compared with that head of the full-shape GPU run;
  * a split-sequence run (two halves, the second starting from the first's
    final state; the first half's backward taking the second half's dh0 /
    dstate0 as its final-state cotangent) equal to the whole run;
  * Mamba2's head-summed dB / dC equal to the sum of single-head runs (the
    head-group reduction of the full shape against runs that have none).
Reference semantics: gdn2_wy_reference.py:105-152 and the B1..B5 chain of
kernel_trainable_B6.py:97-181; mamba2_ssd_reference.py:152-179 and
mamba2_bwd_reference.py:200-266; state passing as kernel_d_pipeline.py:94-124
and kernel_mamba2_c_interchunk.py:38-87.
"""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import gdn2 as G
from atomic_ops import inputs
from atomic_ops import mamba2 as M
from oracle import gdn2 as og
from oracle import mamba2 as om

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

BF16 = torch.bfloat16
T4 = 32768
G_H, G_K, G_C = 16, 128, 64
M_H, M_P, M_N, M_C = 64, 64, 128, 128
HEAD_G = 5     # GDN2 head checked against the oracle
HEAD_M = 37    # Mamba2 head checked against the oracle
# GPU against GPU (the same kernels, a different chunk-loop start): float32
# results to 1e-4; bf16 gradients to the bf16 tolerance (one rounding flip of
# the largest element is 4e-3)
SPLIT_TOL = 1e-4
G_NAMES = ("dq", "dk", "dv", "dw", "db", "dg", "dh0")
M_NAMES = ("ddt", "dx", "dB", "dC", "dA", "dstate0")


def _errs(pairs):
    out = {n: rel_err(a, b) for n, a, b in pairs}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in out.items()), flush=True)
    return out


# ----------------------------------------------------------------------------- GDN2
@pytest.fixture(scope="module")
def gdn2_cfg4():
    banner(f"gdn2 cfg4 full shape B1 T{T4} H{G_H} K=V={G_K} C{G_C}")
    cpu = inputs.gdn2_inputs(1, T4, G_H, G_K, G_K, seed=41, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    args = [dev[n] for n in ("q", "k", "v", "w", "b", "g")]
    o, hf, ws = G.forward(*args, 1.0, save=True)
    grads = G.backward(*args, 1.0, dev["do"], workspace=ws, reuse=True)
    torch.cuda.synchronize()
    del ws
    return cpu, dev, (o, hf), grads


def test_gdn2_cfg4_head_matches_oracle(gdn2_cfg4):
    cpu, _, (o, hf), grads = gdn2_cfg4
    j = HEAD_G
    banner(f"gdn2 cfg4 head {j} against the fp64 oracle (512 chunks)")
    q, k, v, w, b, g, do = (cpu[n][:, :, j:j + 1].contiguous() for n in ("q", "k", "v", "w", "b", "g", "do"))
    o_ref, h_ref = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, G_C)
    ref, _ = og.gdn2_backward_chain(q, k, v, w, b, g, 1.0, G_C, do)
    pairs = [("o", o[:, :, j:j + 1], o_ref), ("h_final", hf[:, j:j + 1], h_ref)]
    pairs += [(n, gr[:, j:j + 1] if n == "dh0" else gr[:, :, j:j + 1], r)
              for n, gr, r in zip(G_NAMES, grads, ref)]
    for n, got, _ in pairs:
        assert torch.isfinite(got).all(), n
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_gdn2_cfg4_split_sequence(gdn2_cfg4):
    """Two halves with h0 = the first half's h_final (forward) and
    dh_final = the second half's dh0 (backward) equal the whole run."""
    _, dev, (o, hf), grads = gdn2_cfg4
    banner("gdn2 cfg4 split sequence")
    half = T4 // 2
    p1 = [dev[n][:, :half].contiguous() for n in ("q", "k", "v", "w", "b", "g", "do")]
    p2 = [dev[n][:, half:].contiguous() for n in ("q", "k", "v", "w", "b", "g", "do")]
    o1, h1, _ = G.forward(*p1[:6], 1.0)
    o2, h2, _ = G.forward(*p2[:6], 1.0, h0=h1)
    g2 = G.backward(*p2[:6], 1.0, p2[6], h0=h1)
    g1 = G.backward(*p1[:6], 1.0, p1[6], dh_final=g2[6])
    torch.cuda.synchronize()
    pairs = [("o", torch.cat([o1, o2], 1), o), ("h_final", h2, hf)]
    pairs += [(n, torch.cat([a, c], 1), whole) for n, a, c, whole in zip(G_NAMES[:6], g1, g2, grads)]
    pairs.append(("dh0", g1[6], grads[6]))
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < (SPLIT_TOL if n in ("o", "h_final", "dg", "dh0") else tol_for(BF16)), (n, e)


def test_gdn2_cfg4_all_finite(gdn2_cfg4):
    _, _, (o, hf), grads = gdn2_cfg4
    for name, t in zip(("o", "h_final") + G_NAMES, (o, hf) + tuple(grads)):
        assert torch.isfinite(t).all(), name


# ----------------------------------------------------------------------------- Mamba2
@pytest.fixture(scope="module")
def mamba2_cfg4():
    banner(f"mamba2 cfg4 full shape B1 T{T4} H{M_H} P{M_P} N{M_N} C{M_C}")
    cpu = inputs.mamba2_inputs(1, T4, M_H, M_P, M_N, seed=43, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    args = [dev[n] for n in ("dt", "x", "Bm", "Cm", "A")]
    y, sf, ws = M.forward(*args, M_C, save=True)
    grads = M.backward(*args, M_C, dev["dy"], workspace=ws, reuse=True)
    torch.cuda.synchronize()
    del ws
    return cpu, dev, (y, sf), grads


def _m2_head(src, j):
    out = {n: src[n][:, :, j:j + 1].contiguous() for n in ("dt", "x", "dy")}
    out.update(Bm=src["Bm"], Cm=src["Cm"], A=src["A"][j:j + 1].contiguous())
    return out


def test_mamba2_cfg4_head_matches_oracle(mamba2_cfg4):
    """Head j of the full-shape run (y, state, ddt, dx, dA, dstate0), and a
    single-head GPU run of the same inputs (whose dB / dC hold that head's
    part only) against the fp64 oracle over 256 chunks."""
    cpu, dev, (y, sf), grads = mamba2_cfg4
    j = HEAD_M
    banner(f"mamba2 cfg4 head {j} against the fp64 oracle (256 chunks)")
    hc = _m2_head(cpu, j)
    y_ref, s_ref = om.mamba2_ssd_reference(hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], M_C)
    ddt_r, dB_r, dC_r, dx_r, dA_r, ds0_r = om.chunk_ssd_bwd_scan(
        hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], M_C, hc["dy"])
    ddt, dx, dB, dC, dA, ds0 = grads
    pairs = [("y", y[:, :, j:j + 1], y_ref), ("state", sf[:, j:j + 1], s_ref),
             ("ddt", ddt[:, :, j:j + 1], ddt_r), ("dx", dx[:, :, j:j + 1], dx_r),
             ("dA", dA[j:j + 1], dA_r), ("dstate0", ds0[:, j:j + 1], ds0_r)]
    hd = _m2_head(dev, j)
    a1 = [hd[n] for n in ("dt", "x", "Bm", "Cm", "A")]
    g1 = M.backward(*a1, M_C, hd["dy"])
    torch.cuda.synchronize()
    pairs += [("dB(head)", g1[2], dB_r), ("dC(head)", g1[3], dC_r)]
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_mamba2_cfg4_head_sum_of_dB_dC(mamba2_cfg4):
    """dB and dC of the full shape (summed over 64 heads in head groups)
    equal the sum of the 64 single-head runs' dB and dC."""
    _, dev, _, grads = mamba2_cfg4
    banner("mamba2 cfg4 dB / dC head sums")
    sB = torch.zeros_like(dev["Bm"], dtype=torch.float32)
    sC = torch.zeros_like(sB)
    for j in range(M_H):
        hd = _m2_head(dev, j)
        g1 = M.backward(*(hd[n] for n in ("dt", "x", "Bm", "Cm", "A")), M_C, hd["dy"])
        sB += g1[2].float()
        sC += g1[3].float()
    torch.cuda.synchronize()
    errs = _errs([("dB", grads[2], sB), ("dC", grads[3], sC)])
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_mamba2_cfg4_split_sequence(mamba2_cfg4):
    _, dev, (y, sf), grads = mamba2_cfg4
    banner("mamba2 cfg4 split sequence")
    half = T4 // 2
    names = ("dt", "x", "Bm", "Cm")
    p1 = [dev[n][:, :half].contiguous() for n in names] + [dev["A"]]
    p2 = [dev[n][:, half:].contiguous() for n in names] + [dev["A"]]
    dy1, dy2 = dev["dy"][:, :half].contiguous(), dev["dy"][:, half:].contiguous()
    y1, s1, _ = M.forward(*p1, M_C)
    y2, s2, _ = M.forward(*p2, M_C, state0=s1)
    g2 = M.backward(*p2, M_C, dy2, state0=s1)
    g1 = M.backward(*p1, M_C, dy1, dstate_final=g2[5])
    torch.cuda.synchronize()
    pairs = [("y", torch.cat([y1, y2], 1), y), ("state", s2, sf)]
    pairs += [(n, torch.cat([a.float(), c.float()], 1), whole)
              for n, a, c, whole in zip(M_NAMES[:4], g1[:4], g2[:4], grads[:4])]
    pairs += [("dA", g1[4] + g2[4], grads[4]), ("dstate0", g1[5], grads[5])]
    errs = _errs(pairs)
    for n, e in errs.items():
        # dA: two partial sums of a near-cancelling reduction, rounded apart
        assert e < (SPLIT_TOL if n in ("y", "state", "dstate0") else tol_for(BF16)), (n, e)


def test_mamba2_cfg4_all_finite(mamba2_cfg4):
    _, _, (y, sf), grads = mamba2_cfg4
    for name, t in zip(("y", "state") + M_NAMES, (y, sf) + tuple(grads)):
        assert torch.isfinite(t).all(), name


# ----------------------------------------------------------------------------- dA drift
@pytest.mark.parametrize("T", [512, 4096])
def test_mamba2_dA_error_against_chunk_count(T):
    """dA is a B*T*P reduction with cancellation whose inputs pass through
    per-chunk states stored in bf16.  Its error at 4 and 32 chunks (the 256
    chunk case is in test_mamba2_cfg4_head_matches_oracle) stays inside the
    bf16 tolerance."""
    H = 4
    banner(f"mamba2 dA drift T{T} H{H}")
    cpu = inputs.mamba2_inputs(1, T, H, M_P, M_N, seed=T + 7, dtype=BF16, dO=True)
    ref = om.chunk_ssd_bwd_scan(cpu["dt"], cpu["A"], cpu["Bm"], cpu["Cm"], cpu["x"], M_C, cpu["dy"])
    dev = {n: t.cuda() for n, t in cpu.items()}
    out = M.backward(*(dev[n] for n in ("dt", "x", "Bm", "Cm", "A")), M_C, dev["dy"])
    torch.cuda.synchronize()
    e = rel_err(out[4], ref[4])
    per_head = ((out[4].cpu().double() - ref[4]).abs() / ref[4].abs()).tolist()
    print(f"  T={T} chunks={T // M_C} dA rel_err={e:.3e} per-head={['%.1e' % x for x in per_head]}",
          flush=True)
    assert e < tol_for(BF16)
