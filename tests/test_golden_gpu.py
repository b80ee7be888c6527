"""The HIP path (through the C ABI) against the committed golden fixtures."""
import os
import sys

import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import gdn2 as G2
from atomic_ops import mamba2 as M2

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu


def _cu(t):
    return None if t is None else t.cuda()


@pytest.mark.parametrize("name", ["gdn2_small.npz", "gdn2_bf16.npz"])
def test_gdn2_matches_fixture(name):
    banner(f"golden {name}")
    f = make_golden.load(name)
    tol = tol_for(f["q"].dtype)
    q, k, v, w, b, g, do = (f[n].cuda() for n in ("q", "k", "v", "w", "b", "g", "do"))
    h0, dht = _cu(f.get("h0")), _cu(f.get("dh_final"))
    o, h, ws = G2.forward(q, k, v, w, b, g, f["scale"], h0=h0, save=True)
    grads = G2.backward(q, k, v, w, b, g, f["scale"], do, dh_final=dht, h0=h0, workspace=ws, reuse=True)
    torch.cuda.synchronize()
    errs = {"o": rel_err(o, f["o"]), "h_final": rel_err(h, f["h_final"])}
    errs.update({n: rel_err(x, f[n]) for n, x in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads)})
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    assert all(e < tol for e in errs.values()), errs


def test_mamba2_matches_fixture():
    banner("golden mamba2_small.npz")
    f = make_golden.load("mamba2_small.npz")
    dt, x, Bm, Cm, A, dy, s0, dsf = (f[n].cuda() for n in ("dt", "x", "Bm", "Cm", "A", "dy", "state0",
                                                          "dstate_final"))
    y, s, ws = M2.forward(dt, x, Bm, Cm, A, f["chunk"], state0=s0, save=True)
    out = M2.backward(dt, x, Bm, Cm, A, f["chunk"], dy, dstate_final=dsf, state0=s0, workspace=ws,
                      reuse=True)
    torch.cuda.synchronize()
    errs = {"y": rel_err(y, f["y"]), "state_final": rel_err(s, f["state_final"])}
    errs.update({n: rel_err(t, f[n]) for n, t in zip(("ddt", "dx", "dB", "dC", "dA", "dstate0"), out)})
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    assert all(e < tol_for(torch.bfloat16) for e in errs.values()), errs
