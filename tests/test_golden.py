"""The committed golden fixtures (tests/golden/, written by make_golden.py
from the float64 oracle) are reproduced by the oracle: guards the oracle
against silent drift once its pinning tests have passed."""
import os
import sys

import pytest
import torch

from _util import rel_err
from oracle import gdn2 as og, mamba2 as om

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden  # noqa: E402

GDN2_OUT = ("dq", "dk", "dv", "dw", "db", "dg", "dh0")


@pytest.mark.parametrize("name", ["gdn2_small.npz", "gdn2_bf16.npz"])
def test_oracle_reproduces_gdn2_fixture(name):
    f = make_golden.load(name)
    h0, dht = f.get("h0"), f.get("dh_final")
    o, h = og.gdn2_chunked_wy_reference(f["q"], f["k"], f["v"], f["g"], f["b"], f["w"], f["scale"],
                                        f["chunk"], h0=h0)
    assert rel_err(o, f["o"]) < 1e-6 and rel_err(h, f["h_final"]) < 1e-6
    grads = og.gdn2_backward_autodiff(f["q"], f["k"], f["v"], f["w"], f["b"], f["g"], f["scale"],
                                      f["chunk"], f["do"], dh_final=dht, h0=h0)
    for n, gr in zip(GDN2_OUT, grads):
        assert rel_err(gr, f[n]) < 1e-6, n


def test_oracle_reproduces_mamba2_fixture():
    f = make_golden.load("mamba2_small.npz")
    y, s = om.mamba2_ssd_reference(f["dt"], f["A"], f["Bm"], f["Cm"], f["x"], f["chunk"],
                                   state0=f["state0"])
    assert rel_err(y, f["y"]) < 1e-6 and rel_err(s, f["state_final"]) < 1e-6
    out = om.chunk_ssd_bwd_scan(f["dt"], f["A"], f["Bm"], f["Cm"], f["x"], f["chunk"], f["dy"],
                                f["dstate_final"], state0=f["state0"])
    for n, gr in zip(("ddt", "dB", "dC", "dx", "dA", "dstate0"), out):
        assert rel_err(gr, f[n]) < 1e-6, n


def test_fixture_inputs_follow_the_benchmark_distributions():
    f = make_golden.load("gdn2_small.npz")
    assert torch.allclose(f["q"].double().norm(dim=-1), torch.ones(1, dtype=torch.float64), atol=1e-5)
    assert (f["g"] < 0).all() and (f["b"] > 0).all() and (f["b"] < 1).all()
    m = make_golden.load("mamba2_small.npz")
    assert (m["A"] < 0).all() and (m["dt"].float() > 0).all()
