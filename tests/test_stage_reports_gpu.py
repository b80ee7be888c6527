"""Per-stage reports (the args structs' `diag`; the reference's opt-in
GDN2_FWD_DIAG stage check, kernel_d_pipeline.py:50-91) on the GPU, and the
clip / nan_to_num placement on inputs that make it fire (the reference's
failure handling: NaN, +-inf and beyond-1e4 inputs return its sanitised
values).

Each report must equal the non-finite count and max |x| of the same stage
in the float64 oracle: the GDN2 stages of gdn2_wy_reference.py:59-152 and the
B1..B5 chain's intermediates; the Mamba2 stages of mamba2_ssd_reference.py
and the MB0 reverse scan."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import _lib
from atomic_ops import gdn2 as G
from atomic_ops import inputs
from atomic_ops import mamba2 as M
from oracle import gdn2 as og
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32
GN = ("q", "k", "v", "w", "b", "g")


def _stat(ts):
    """(non-finite count, max |x| of the finite part) of a tensor or list."""
    if isinstance(ts, (list, tuple)):
        ts = torch.stack([t.double() for t in ts])
    ts = ts.detach().double().cpu()
    fin = torch.isfinite(ts)
    return int((~fin).sum()), (ts[fin].abs().max().item() if fin.any() else 0.0)


def _compare(rep, ref, tol):
    bad = []
    for name, (n_ref, m_ref) in ref.items():
        n_got, m_got = rep[name]
        print(f"  {name:22s} nonfinite {n_got} (oracle {n_ref})  max {m_got:.4e} (oracle {m_ref:.4e})")
        if n_got != n_ref or abs(m_got - m_ref) > tol * max(m_ref, 1e-30):
            bad.append(name)
    assert not bad, bad


def _gdn2_reference_stats(cpu, h0=None, dh=None, scale=1.0):
    q, k, v, w, b, g, do = (cpu[n] for n in GN + ("do",))
    o, h, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 64, h0=h0, return_stages=True)
    grads, inter = og.gdn2_backward_chain(q, k, v, w, b, g, scale, 64, do, dh, h0=h0)
    fwd = {name: _stat([s[key] for s in st]) for name, key in zip(
        _lib.GDN2_DIAG_STAGES[:7], ("Aqk", "Akk", "A", "w_pseudo", "u", "kg", "qg"))}
    fwd["kernel_D_o"], fwd["kernel_D_h_final"] = _stat(o), _stat(h)
    bwd = {"bwd_dv_new": _stat(inter["dv_new"]), "bwd_dh": _stat(inter["dh_next"]),
           "bwd_dAqk": _stat([scale * x for x in inter["dAqk"]]), "bwd_dAkk": _stat(inter["dAkk"])}
    bwd.update({n: _stat(gr) for n, gr in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads)})
    return (o, h), grads, fwd, bwd


@pytest.mark.parametrize("dtype,K", [(BF16, 128), (F32, 64)])
def test_gdn2_reports_equal_the_oracle_stages(dtype, K):
    banner(f"gdn2 stage reports {dtype} K{K}")
    cpu = inputs.gdn2_inputs(1, 192, 2, K, K, seed=51, dtype=dtype, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    rep = _lib.StageReports(_lib.GDN2_DIAG_STAGES, "cuda")
    _, _, ws = G.forward(*(dev[n] for n in GN), 1.0, save=True, diag=rep)
    G.backward(*(dev[n] for n in GN), 1.0, dev["do"], workspace=ws, reuse=True, diag=rep)
    _, _, fwd, bwd = _gdn2_reference_stats(cpu)
    got = rep.read()
    _compare(got, fwd, tol_for(dtype))
    _compare(got, bwd, tol_for(dtype))


def test_gdn2_reports_off_by_default_and_repeatable():
    """No report buffer: nothing is written (the outputs are the same as
    with reports).  With one: each call clears what it covers first."""
    banner("gdn2 stage reports cleared per call")
    d = inputs.gdn2_inputs(1, 128, 2, 64, 64, seed=52, dtype=F32, device="cuda")
    args = [d[n] for n in GN]
    o1, h1, _ = G.forward(*args, 1.0)
    rep = _lib.StageReports(_lib.GDN2_DIAG_STAGES, "cuda")
    rep.buf.fill_(7)
    o2, h2, _ = G.forward(*args, 1.0, diag=rep)
    o3, _, _ = G.forward(*args, 1.0, diag=rep)
    assert torch.equal(o1, o2) and torch.equal(h1, h2) and torch.equal(o2, o3)
    got = rep.read()
    assert all(got[n][0] == 0 for n in _lib.GDN2_DIAG_STAGES[:_lib.GDN2_DIAG_FWD])
    # the backward's entries were not touched by the forward
    assert rep.buf[_lib.GDN2_DIAG_FWD:].eq(7).all()


def _poison(cpu):
    q, v = cpu["q"], cpu["v"]
    q[0, 10, 0, 3] = float("nan")
    q[0, 75, 1, 9] = float("inf")
    q[0, 140, 0, 0] = -float("inf")
    v[0, 20:24, 1, :] = 3e4


def test_gdn2_forward_sanitises_nonfinite_and_large_inputs():
    """NaN / +-inf in q (through Aqk, qg and o) and beyond-1e4 values in v
    and h0 (through u, v_new, o and the state clip): o and h_final equal the
    oracle's sanitised values, and the reports count the non-finite qg
    entries the reference function keeps (gdn2_wy_reference.py:100)."""
    banner("gdn2 forward on NaN / inf / large inputs")
    cpu = inputs.gdn2_inputs(1, 192, 2, 64, 64, seed=5, dtype=F32, dO=True)
    _poison(cpu)
    h0 = torch.zeros(1, 2, 64, 64)
    h0[0, 0, :4, :] = 2e4
    dev = {n: t.cuda() for n, t in cpu.items()}
    rep = _lib.StageReports(_lib.GDN2_DIAG_STAGES, "cuda")
    o, hf, _ = G.forward(*(dev[n] for n in GN), 1.0, h0=h0.cuda(), diag=rep)
    q, k, v, w, b, g = (cpu[n] for n in GN)
    o_ref, h_ref, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 64, h0=h0, return_stages=True)
    eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
    print(f"  rel_err o={eo:.2e} h_final={eh:.2e}")
    assert torch.isfinite(o).all() and torch.isfinite(hf).all()
    assert eo < tol_for(F32) and eh < tol_for(F32)
    got = rep.read()
    assert got["kernel_C_qg"][0] == _stat([s["qg"] for s in st])[0] == 3
    for name in ("kernel_A_Aqk", "kernel_C_u", "kernel_D_o", "kernel_D_h_final"):
        assert got[name][0] == 0, name
    assert abs(got["kernel_A_Aqk"][1] - 1e4) < 1.0          # +-inf q . k -> n2n -> 1e4
    assert got["kernel_D_o"][1] > 1e4 * 0.99                 # the 3e4 values of v reach o


def test_gdn2_backward_with_clips_firing():
    """Beyond-1e4 v, h0 and dh_final: the backward's straight-through clip
    masks (B1's dh and dv_new sanitise, the final clip) fire; gradients
    equal the oracle's."""
    banner("gdn2 backward with clips firing")
    cpu = inputs.gdn2_inputs(1, 192, 2, 64, 64, seed=6, dtype=F32, dO=True)
    cpu["v"][0, 20:24, 1, :] = 3e4
    h0 = torch.zeros(1, 2, 64, 64)
    h0[0, 0, :4, :] = 2e4
    dh = torch.randn(1, 2, 64, 64, generator=torch.Generator().manual_seed(3)) * 5e3
    dev = {n: t.cuda() for n, t in cpu.items()}
    rep = _lib.StageReports(_lib.GDN2_DIAG_STAGES, "cuda")
    grads = G.backward(*(dev[n] for n in GN), 1.0, dev["do"], dh_final=dh.cuda(), h0=h0.cuda(), diag=rep)
    _, ref, _, bwd = _gdn2_reference_stats(cpu, h0=h0, dh=dh)
    errs = {n: rel_err(a, r) for n, a, r in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads, ref)}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for n, e in errs.items():
        assert e < tol_for(F32), (n, e)
    _compare(rep.read(), bwd, tol_for(F32))


def _mamba2_reference_stats(cpu, C):
    dt, x, Bm, Cm, A, dy = (cpu[n] for n in ("dt", "x", "Bm", "Cm", "A", "dy"))
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    chunks = [om._to_chunks(t, C) for t in (dt, Bm, Cm, x, dy)]
    state = torch.zeros(b, h, p, n, dtype=torch.float64)
    states, cbs, ys = [], [], []
    for c in range(l // C):
        states.append(state)
        y_c, state, parts = om.chunk_ssd(chunks[0][c], A, chunks[1][c], chunks[2][c], chunks[3][c], state)
        cbs.append(parts["CB"])
        ys.append(y_c)
    fwd = {"cb": _stat(cbs), "chunk_states": _stat(states), "ssm_out": _stat(ys), "state_final": _stat(state)}
    dstate = torch.zeros_like(state)
    dstates = []
    for c in reversed(range(l // C)):
        dstates.append(dstate)
        *_, dstate, _ = om.chunk_ssd_bwd(chunks[0][c], A, chunks[1][c], chunks[2][c], chunks[3][c], states[c],
                                         chunks[4][c], dstate)
    grads = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy)
    bwd = {"bwd_dstates": _stat(dstates)}
    bwd.update({nm: _stat(gr) for nm, gr in zip(("ddt", "dB", "dC", "dx", "dA", "dstate0"), grads)})
    return fwd, bwd


def test_mamba2_reports_and_clips_equal_the_oracle():
    """Reports of every Mamba2 stage, with x large enough that the 1e4
    sanitise of dt x fires (and its straight-through mask in the backward,
    whose ddt / dB / dC then reach the final 1e4 clip): outputs, gradients
    and reports equal the oracle's."""
    banner("mamba2 stage reports, clips firing")
    C = 128
    cpu = inputs.mamba2_inputs(1, 512, 4, 64, 128, seed=53, dtype=BF16, dO=True)
    cpu["x"][0, 100:104, 2, :] = 3e5      # dt x ~ 4e4: sanitize(dt x, 1e4) fires
    dev = {n: t.cuda() for n, t in cpu.items()}
    rep = _lib.StageReports(_lib.MAMBA2_DIAG_STAGES, "cuda")
    args = [dev[n] for n in ("dt", "x", "Bm", "Cm", "A")]
    y, sf, ws = M.forward(*args, C, save=True, diag=rep)
    grads = M.backward(*args, C, dev["dy"], workspace=ws, reuse=True, diag=rep)
    dt, x, Bm, Cm, A, dy = (cpu[n] for n in ("dt", "x", "Bm", "Cm", "A", "dy"))
    y_ref, s_ref = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C)
    ddt_r, dB_r, dC_r, dx_r, dA_r, ds0_r = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy)
    errs = {n: rel_err(a, r) for n, a, r in zip(
        ("y", "state", "ddt", "dx", "dB", "dC", "dA", "dstate0"), (y, sf) + tuple(grads),
        (y_ref, s_ref, ddt_r, dx_r, dB_r, dC_r, dA_r, ds0_r))}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    assert (dt.float() * x.float()).abs().max() > 1e4      # dBx's sanitise fires
    assert ddt_r.abs().max().item() == pytest.approx(1e4)  # and the final clip of ddt
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)
    fwd, bwd = _mamba2_reference_stats(cpu, C)
    got = rep.read()
    _compare(got, fwd, tol_for(BF16))
    _compare(got, bwd, tol_for(BF16))
