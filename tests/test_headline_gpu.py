"""The benchmark's own shape (B4 T8192 H16, d = 128) through the kernel forms
that shape selects, checked at full length on the GPU.

At B4 H16 the GDN2 state loops take their 32-column V tiles (B*H*V/16 > 256):
the forward loop at sixteen waves with one register prefetch set, the dh loop
with two LDS stage buffers and its dv_new tiles written one step late.  The
Mamba2 chunk kernels at P = N = 128 take their multi-pair forms (16 (head,
slice) pairs per chunk_y workgroup, 8 per chunk_outer workgroup, two 8-head
groups in the chunk backward).  Each path is checked three ways at the full
shape, as the long-context tests do:
  * two (batch, head) units of the full-shape run against the float64 oracle,
    forward and backward (dA included);
  * a split-sequence run (two halves, state and state cotangent handed over)
    against the whole run;
  * Mamba2's head-summed dB / dC against the sum of single-head runs.
A smaller case runs the 32-column loops over 8 chunks at B1 H48, with and
without h0, against the oracle and bit for bit against the 16-column loops
(the same heads in two calls of 24, where B*H*V/16 <= 256): every output
element is the same sequence of MFMA steps in both, only the tile width
differs.
Reference semantics: gdn2_wy_reference.py:105-152 and the B1..B5 chain of
kernel_trainable_B6.py:97-181 (its meaning: kernel_trainable.py:38-55);
mamba2_ssd_reference.py:152-179 and mamba2_bwd_reference.py:200-266.
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
B, T, H = 4, 8192, 16
G_K, G_C = 128, 64
M_P, M_N, M_C = 128, 128, 128
UNITS = ((1, 3), (3, 12))   # (batch row, head) units checked against the oracle
SPLIT_TOL = 1e-4            # GPU against GPU, float32 results
G_NAMES = ("dq", "dk", "dv", "dw", "db", "dg", "dh0")
M_NAMES = ("ddt", "dx", "dB", "dC", "dA", "dstate0")
GIN = ("q", "k", "v", "w", "b", "g")


def _errs(pairs):
    out = {n: rel_err(a, b) for n, a, b in pairs}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in out.items()), flush=True)
    return out


# ----------------------------------------------------------------------------- GDN2
@pytest.fixture(scope="module")
def gdn2_head():
    banner(f"gdn2 headline full shape B{B} T{T} H{H} K=V={G_K} C{G_C}")
    cpu = inputs.gdn2_inputs(B, T, H, G_K, G_K, seed=61, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    args = [dev[n] for n in GIN]
    o, hf, ws = G.forward(*args, 1.0, save=True)
    grads = G.backward(*args, 1.0, dev["do"], workspace=ws, reuse=True)
    torch.cuda.synchronize()
    del ws
    return cpu, dev, (o, hf), grads


@pytest.mark.parametrize("unit", UNITS)
def test_gdn2_headline_unit_matches_oracle(gdn2_head, unit):
    cpu, _, (o, hf), grads = gdn2_head
    bb, j = unit
    banner(f"gdn2 headline unit b{bb} h{j} against the fp64 oracle (128 chunks)")
    sl = lambda t: t[bb:bb + 1, :, j:j + 1].contiguous()
    q, k, v, w, b, g, do = (sl(cpu[n]) for n in GIN + ("do",))
    o_ref, h_ref = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, G_C)
    ref, _ = og.gdn2_backward_chain(q, k, v, w, b, g, 1.0, G_C, do)
    pairs = [("o", o[bb:bb + 1, :, j:j + 1], o_ref), ("h_final", hf[bb:bb + 1, j:j + 1], h_ref)]
    pairs += [(n, gr[bb:bb + 1, j:j + 1] if n == "dh0" else gr[bb:bb + 1, :, j:j + 1], r)
              for n, gr, r in zip(G_NAMES, grads, ref)]
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_gdn2_headline_split_sequence(gdn2_head):
    """Two halves (64 chunks each, the same 32-column loops) with the state
    and its cotangent handed over equal the whole run."""
    _, dev, (o, hf), grads = gdn2_head
    banner("gdn2 headline split sequence")
    half = T // 2
    p1 = [dev[n][:, :half].contiguous() for n in GIN + ("do",)]
    p2 = [dev[n][:, half:].contiguous() for n in GIN + ("do",)]
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


def test_gdn2_headline_all_finite(gdn2_head):
    _, _, (o, hf), grads = gdn2_head
    for name, t in zip(("o", "h_final") + G_NAMES, (o, hf) + tuple(grads)):
        assert torch.isfinite(t).all(), name


@pytest.mark.parametrize("with_h0", [False, True])
def test_gdn2_wide_tile_loops_over_many_chunks(with_h0):
    """B1 T512 H48 (8 chunks, B*H*V/16 = 384: the 32-column loops) against the
    oracle for every head, and bit for bit against the 16-column loops (heads
    0-23 and 24-47 as two calls, B*H*V/16 = 192)."""
    Hh, Tt = 48, 512
    banner(f"gdn2 32-column loops B1 T{Tt} H{Hh} h0={with_h0}")
    cpu = inputs.gdn2_inputs(1, Tt, Hh, G_K, G_K, seed=67, dtype=BF16, dO=True)
    gen = torch.Generator().manual_seed(68)
    h0 = torch.randn(1, Hh, G_K, G_K, generator=gen) if with_h0 else None
    dhf = torch.randn(1, Hh, G_K, G_K, generator=gen) if with_h0 else None
    dev = {n: t.cuda() for n, t in cpu.items()}
    h0d = h0.cuda() if with_h0 else None
    dhfd = dhf.cuda() if with_h0 else None
    args = [dev[n] for n in GIN]
    o, hf, ws = G.forward(*args, 1.0, h0=h0d, save=True)
    grads = G.backward(*args, 1.0, dev["do"], dh_final=dhfd, h0=h0d, workspace=ws, reuse=True)
    # the same heads in two calls of 24 (row-strided head slices, read in place)
    parts = []
    for h_lo in (0, 24):
        sl = lambda t: t[:, :, h_lo:h_lo + 24]
        a2 = [sl(dev[n]) for n in GIN]
        hh = h0d[:, h_lo:h_lo + 24].contiguous() if with_h0 else None
        dd = dhfd[:, h_lo:h_lo + 24].contiguous() if with_h0 else None
        o2, hf2, ws2 = G.forward(*a2, 1.0, h0=hh, save=True)
        g2 = G.backward(*a2, 1.0, sl(dev["do"]), dh_final=dd, h0=hh, workspace=ws2, reuse=True)
        parts.append((o2, hf2, g2))
    torch.cuda.synchronize()
    o16 = torch.cat([p[0] for p in parts], 2)
    hf16 = torch.cat([p[1] for p in parts], 1)
    g16 = [torch.cat([p[2][i] for p in parts], 1 if i == 6 else 2) for i in range(7)]
    for n, a, c in zip(("o", "h_final") + G_NAMES, (o, hf) + tuple(grads), (o16, hf16) + tuple(g16)):
        assert torch.equal(a, c), f"{n}: 32-column and 16-column loops differ"
    o_ref, h_ref = og.gdn2_chunked_wy_reference(*(cpu[n] for n in ("q", "k", "v", "g", "b", "w")), 1.0, G_C,
                                                h0=h0)
    ref, _ = og.gdn2_backward_chain(*(cpu[n] for n in GIN), 1.0, G_C, cpu["do"], dhf, h0=h0)
    errs = _errs([("o", o, o_ref), ("h_final", hf, h_ref)] + list(zip(G_NAMES, grads, ref)))
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


# ----------------------------------------------------------------------------- Mamba2
@pytest.fixture(scope="module")
def mamba2_head():
    banner(f"mamba2 headline full shape B{B} T{T} H{H} P{M_P} N{M_N} C{M_C}")
    cpu = inputs.mamba2_inputs(B, T, H, M_P, M_N, seed=63, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    args = [dev[n] for n in ("dt", "x", "Bm", "Cm", "A")]
    y, sf, ws = M.forward(*args, M_C, save=True)
    grads = M.backward(*args, M_C, dev["dy"], workspace=ws, reuse=True)
    torch.cuda.synchronize()
    del ws
    return cpu, dev, (y, sf), grads


def _m2_unit(src, bb, j):
    out = {n: src[n][bb:bb + 1, :, j:j + 1].contiguous() for n in ("dt", "x", "dy")}
    out.update(Bm=src["Bm"][bb:bb + 1].contiguous(), Cm=src["Cm"][bb:bb + 1].contiguous(),
               A=src["A"][j:j + 1].contiguous())
    return out


@pytest.mark.parametrize("unit", UNITS)
def test_mamba2_headline_unit_matches_oracle(mamba2_head, unit):
    """Unit (b, h) of the full-shape run (y, state, ddt, dx, dstate0) and a
    one-unit GPU run of the same inputs (whose dB / dC / dA hold that unit's
    part only) against the fp64 oracle over 64 chunks."""
    cpu, dev, (y, sf), grads = mamba2_head
    bb, j = unit
    banner(f"mamba2 headline unit b{bb} h{j} against the fp64 oracle (64 chunks)")
    hc = _m2_unit(cpu, bb, j)
    y_ref, s_ref = om.mamba2_ssd_reference(hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], M_C)
    ddt_r, dB_r, dC_r, dx_r, dA_r, ds0_r = om.chunk_ssd_bwd_scan(
        hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], M_C, hc["dy"])
    ddt, dx, dB, dC, dA, ds0 = grads
    pairs = [("y", y[bb:bb + 1, :, j:j + 1], y_ref), ("state", sf[bb:bb + 1, j:j + 1], s_ref),
             ("ddt", ddt[bb:bb + 1, :, j:j + 1], ddt_r), ("dx", dx[bb:bb + 1, :, j:j + 1], dx_r),
             ("dstate0", ds0[bb:bb + 1, j:j + 1], ds0_r)]
    hd = _m2_unit(dev, bb, j)
    g1 = M.backward(*(hd[n] for n in ("dt", "x", "Bm", "Cm", "A")), M_C, hd["dy"])
    torch.cuda.synchronize()
    pairs += [("dB(unit)", g1[2], dB_r), ("dC(unit)", g1[3], dC_r), ("dA(unit)", g1[4], dA_r)]
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


@pytest.mark.parametrize("j", [UNITS[0][1], UNITS[1][1]])
def test_mamba2_headline_dA_matches_oracle(mamba2_head, j):
    """dA[j] of the full run sums over the four batch rows (the batch part of
    the reduction).  The rows' own dA cancel (head 12 of this input: +0.63,
    -1.41, +0.17, +0.57 sum to -0.036), so the error of the sum is measured
    against the largest row term, the norm-wise metric over the terms the
    reduction adds; the error against the sum itself is printed as well."""
    cpu, _, _, grads = mamba2_head
    banner(f"mamba2 headline dA[{j}] over {B} batch rows against the fp64 oracle")
    rows = []
    for bb in range(B):
        hc = _m2_unit(cpu, bb, j)
        rows.append(om.chunk_ssd_bwd_scan(hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], M_C, hc["dy"])[4])
    ref = sum(rows)
    got = grads[4][j:j + 1].cpu().double()
    scale = max(r.abs().max().item() for r in rows)
    e_terms = (got - ref).abs().max().item() / scale
    print(f"  dA[{j}]={got.item():.5f} oracle={ref.item():.5f} rows={[round(r.item(), 4) for r in rows]} "
          f"err/max|row|={e_terms:.2e} err/|sum|={rel_err(got, ref):.2e}", flush=True)
    assert e_terms < tol_for(BF16)


def test_mamba2_headline_head_sum_of_dB_dC(mamba2_head):
    """dB and dC of the full shape (summed over 16 heads in two head groups)
    equal the sum of the 16 single-head runs' dB and dC."""
    _, dev, _, grads = mamba2_head
    banner("mamba2 headline dB / dC head sums")
    sB = torch.zeros_like(dev["Bm"], dtype=torch.float32)
    sC = torch.zeros_like(sB)
    for j in range(H):
        hd = {n: dev[n][:, :, j:j + 1].contiguous() for n in ("dt", "x", "dy")}
        g1 = M.backward(hd["dt"], hd["x"], dev["Bm"], dev["Cm"], dev["A"][j:j + 1].contiguous(), M_C, hd["dy"])
        sB += g1[2].float()
        sC += g1[3].float()
    torch.cuda.synchronize()
    errs = _errs([("dB", grads[2], sB), ("dC", grads[3], sC)])
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_mamba2_headline_split_sequence(mamba2_head):
    _, dev, (y, sf), grads = mamba2_head
    banner("mamba2 headline split sequence")
    half = T // 2
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
        assert e < (SPLIT_TOL if n in ("y", "state", "dstate0") else tol_for(BF16)), (n, e)


def test_mamba2_headline_all_finite(mamba2_head):
    _, _, (y, sf), grads = mamba2_head
    for name, t in zip(("y", "state") + M_NAMES, (y, sf) + tuple(grads)):
        assert torch.isfinite(t).all(), name
