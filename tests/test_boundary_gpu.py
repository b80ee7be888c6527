"""Drop-in boundary details of the whole-path entries on the GPU.

* The trainable ops sanitise the initial state like the reference's staged
  forward (h0: _sanitize_h0, kernel_d_pipeline.py:54-55,101, run by
  kernel_trainable_B6.py:87-88; state0: kernel_mamba2_c_interchunk.py:56-58,
  run by kernel_mamba2_trainable_B6.py:72-80): with h0 / state0 beyond +-1e4
  and NaN they equal the oracle fed the sanitised state, and the plain
  entries (no flag) equal the oracle fed the raw state.
* The REUSE record holds the query scale (folded into the saved Aqk) and the
  sanitise flag: a backward that differs in either is refused.
* The trainable ops recompute when the library no longer holds the saving
  forward's record (the table keeps the newest 1024 records).
"""
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

BF16 = torch.bfloat16
GIN = ("q", "k", "v", "w", "b", "g")
MIN = ("dt", "x", "Bm", "Cm", "A")


def _wild_state(shape, seed):
    """A state with entries at +-2e4, NaN and +-inf among ordinary ones."""
    gen = torch.Generator().manual_seed(seed)
    s = torch.randn(*shape, generator=gen)
    s[0, 0, :4, :] = 2e4
    s[0, 0, 4:6, :] = -3e4
    s[0, -1, 0, :8] = float("nan")
    s[0, -1, 1, :8] = float("inf")
    s[0, -1, 2, :8] = float("-inf")
    return s


def _sanitized(s):
    return torch.nan_to_num(s.clamp(-1e4, 1e4), nan=0.0, posinf=1e4, neginf=-1e4)


def test_gdn2_trainable_sanitises_h0():
    from atomic_ops.kernel_trainable_B6 import gdn2_pallas_forward_trainable
    Bb, T, H, K = 1, 128, 2, 64
    banner("gdn2 trainable op with h0 beyond 1e4 / NaN / inf")
    cpu = inputs.gdn2_inputs(Bb, T, H, K, K, seed=71, dtype=BF16, dO=True)
    h0 = _wild_state((Bb, H, K, K), 72)
    dev = {n: t.cuda() for n, t in cpu.items()}
    leaves = [dev[n].clone().requires_grad_(True) for n in GIN]
    h0l = h0.cuda().requires_grad_(True)
    o, hf = gdn2_pallas_forward_trainable(*leaves, 1.0, h0l)
    (o * dev["do"].float()).sum().backward()
    torch.cuda.synchronize()
    hs = _sanitized(h0)
    o_ref, h_ref = og.gdn2_chunked_wy_reference(*(cpu[n] for n in ("q", "k", "v", "g", "b", "w")), 1.0, 64,
                                                h0=hs)
    ref, _ = og.gdn2_backward_chain(*(cpu[n] for n in GIN), 1.0, 64, cpu["do"], h0=hs)
    got = [t.grad for t in leaves] + [h0l.grad]
    errs = {n: rel_err(a, r) for n, a, r in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), got, ref)}
    errs.update(o=rel_err(o, o_ref), h_final=rel_err(hf, h_ref))
    print("  rel_err " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)
    # the plain entry takes h0 as given (gdn2_chunked_wy_reference): a state
    # of +-2e4 decays for a chunk before the state clip, so o differs
    o_raw, _, _ = G.forward(*(dev[n] for n in GIN), 1.0, h0=torch.nan_to_num(h0, nan=0.0, posinf=0.0,
                                                                              neginf=0.0).cuda())
    torch.cuda.synchronize()
    assert not torch.allclose(o_raw, o)


def test_mamba2_trainable_sanitises_state0():
    from atomic_ops.kernel_mamba2_trainable_B6 import mamba2_pallas_forward_trainable_B6
    Bb, T, H, P, N = 1, 256, 2, 64, 128
    banner("mamba2 trainable op with state0 beyond 1e4 / NaN / inf")
    cpu = inputs.mamba2_inputs(Bb, T, H, P, N, seed=73, dtype=BF16, dO=True)
    s0 = _wild_state((Bb, H, P, N), 74)
    dev = {n: t.cuda() for n, t in cpu.items()}
    leaves = [dev[n].clone().requires_grad_(True) for n in MIN]
    s0l = s0.cuda().requires_grad_(True)
    y, sf = mamba2_pallas_forward_trainable_B6(*leaves[:4], leaves[4], 128, s0l)
    (y * dev["dy"].float()).sum().backward()
    torch.cuda.synchronize()
    ss = _sanitized(s0)
    y_ref, s_ref = om.mamba2_ssd_reference(cpu["dt"], cpu["A"], cpu["Bm"], cpu["Cm"], cpu["x"], 128, state0=ss)
    ref = om.chunk_ssd_bwd_scan(cpu["dt"], cpu["A"], cpu["Bm"], cpu["Cm"], cpu["x"], 128, cpu["dy"], state0=ss)
    ddt_r, dB_r, dC_r, dx_r, dA_r, ds0_r = ref
    got = dict(zip(("ddt", "dx", "dB", "dC", "dA"), (t.grad for t in leaves)))
    errs = {"y": rel_err(y, y_ref), "state": rel_err(sf, s_ref), "ddt": rel_err(got["ddt"], ddt_r),
            "dx": rel_err(got["dx"], dx_r), "dB": rel_err(got["dB"], dB_r), "dC": rel_err(got["dC"], dC_r),
            "dA": rel_err(got["dA"], dA_r), "dstate0": rel_err(s0l.grad, ds0_r)}
    print("  rel_err " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_reuse_record_holds_scale_and_sanitise_flag():
    banner("gdn2 / mamba2 reuse record: scale and sanitise flag")
    cpu = inputs.gdn2_inputs(1, 128, 2, 64, 64, seed=75, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    a = [dev[n] for n in GIN]
    _, _, ws = G.forward(*a, 0.5, save=True)
    with pytest.raises(_lib.AtomicError, match="REUSE"):
        G.backward(*a, 1.0, dev["do"], workspace=ws, reuse=True)
    with pytest.raises(_lib.AtomicError, match="REUSE"):
        G.backward(*a, 0.5, dev["do"], workspace=ws, reuse=True, sanitize_h0=True)
    got = G.backward(*a, 0.5, dev["do"], workspace=ws, reuse=True)
    want = G.backward(*a, 0.5, dev["do"])
    torch.cuda.synchronize()
    for x, y in zip(got, want):
        assert torch.equal(x, y)
    m = inputs.mamba2_inputs(1, 256, 2, 64, 128, seed=76, dtype=BF16, dO=True)
    md = {n: t.cuda() for n, t in m.items()}
    ma = [md[n] for n in MIN]
    _, _, mws = M.forward(*ma, 128, save=True, sanitize_state0=True)
    with pytest.raises(_lib.AtomicError, match="REUSE"):
        M.backward(*ma, 128, md["dy"], workspace=mws, reuse=True)
    M.backward(*ma, 128, md["dy"], workspace=mws, reuse=True, sanitize_state0=True)
    torch.cuda.synchronize()


def test_trainable_ops_recompute_when_the_record_is_gone():
    """1024 further saving forwards push the trainable op's record out of the
    table; its backward then recomputes and gives the same gradients."""
    from atomic_ops.kernel_mamba2_trainable_B6 import mamba2_pallas_forward_trainable_B6
    from atomic_ops.kernel_trainable_B6 import gdn2_pallas_forward_trainable
    banner("trainable ops after their REUSE record is evicted")
    cpu = inputs.gdn2_inputs(1, 64, 1, 64, 64, seed=77, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    m = inputs.mamba2_inputs(1, 64, 1, 64, 64, seed=78, dtype=BF16, dO=True)
    md = {n: t.cuda() for n, t in m.items()}

    def gdn2_grads():
        leaves = [dev[n].clone().requires_grad_(True) for n in GIN]
        o, _ = gdn2_pallas_forward_trainable(*leaves, 1.0)
        return o, leaves

    def mamba2_grads():
        leaves = [md[n].clone().requires_grad_(True) for n in MIN]
        y, _ = mamba2_pallas_forward_trainable_B6(*leaves[:4], leaves[4], 64)
        return y, leaves

    o, gl = gdn2_grads()
    y, ml = mamba2_grads()
    keep = []
    for i in range(1030):   # distinct live workspaces, each recorded
        _, _, ws = G.forward(*(dev[n] for n in GIN), 1.0, save=True)
        keep.append(ws)
    (o * dev["do"].float()).sum().backward()
    (y * md["dy"].float()).sum().backward()
    o2, gl2 = gdn2_grads()
    y2, ml2 = mamba2_grads()
    (o2 * dev["do"].float()).sum().backward()
    (y2 * md["dy"].float()).sum().backward()
    torch.cuda.synchronize()
    for a, c in zip(gl + ml, gl2 + ml2):
        assert torch.equal(a.grad, c.grad)
