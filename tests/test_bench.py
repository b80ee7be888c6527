"""Host-side checks of bench.py (no GPU): the one-GPU guard, the algorithmic
byte / flop models that the roofline figures divide by, and the reading of
the committed counter summary."""
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line


@pytest.mark.parametrize("model", ["gdn2", "mamba2"])
def test_kernel_models_are_linear_in_batch_and_sequence(model):
    b = _bench()
    if model == "gdn2":
        f = lambda B, T: b.gdn2_kernel_model(B, T, 16, 128, 128, 64)
    else:
        f = lambda B, T: b.mamba2_kernel_model(B, T, 16, 128, 128, 128)
    one, two_b, two_t = f(1, 2048), f(2, 2048), f(1, 4096)
    assert set(one) == set(two_b) == set(two_t)
    for k in one:
        fl, by = one[k]
        assert fl >= 0 and by > 0, k
        # per (batch, head, chunk) units: doubling the batch doubles everything
        assert two_b[k][1] == pytest.approx(2 * by, rel=1e-5), k
        assert two_b[k][0] == pytest.approx(2 * fl, rel=1e-5), k
        # doubling the sequence doubles the per-chunk terms; the per-sequence
        # ones (initial / final state of the state passes) stay, so the
        # ratio lies just below 2
        assert 1.85 * by <= two_t[k][1] <= 2 * by * (1 + 1e-9), k
        assert two_t[k][0] == pytest.approx(2 * fl, rel=1e-5), k


def test_roofline_picks_the_bound_by_arithmetic_intensity():
    b = _bench()
    nbytes, sec = 1e9, 1e-3
    lo = b.roofline(flops=0.1 * b.RIDGE * nbytes, nbytes=nbytes, seconds=sec)
    hi = b.roofline(flops=10 * b.RIDGE * nbytes, nbytes=nbytes, seconds=sec)
    assert lo["bound"] == "hbm" and lo["unit"] == "GB/s"
    assert lo["achieved"] == pytest.approx(nbytes / sec / 1e9)
    assert lo["frac"] == pytest.approx(lo["achieved"] / lo["peak"])
    assert hi["bound"] == "mfma" and hi["unit"] == "TFLOP/s"
    assert hi["frac"] == pytest.approx(hi["achieved"] / hi["peak"])


def test_measured_traffic_reads_the_committed_summary():
    b = _bench()
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        t = json.load(f)
    assert b.measured_traffic(t["kernel"]) == int(t["bytes_per_launch"])
    assert b.measured_traffic("not_a_kernel") is None


def test_path_model_reproduces_the_measurement_plan_figures():
    """The path-level model gives the figures the measurement plan states:
    GDN2 at configurations 2 / 3 fwd 95.2 GFLOP / 1.21 GB and bwd 197.6 GFLOP /
    2.01 GB; Mamba2 forward at configuration 1 13.2 GFLOP / 138 MB; the
    headline Mamba2 forward 100.4 kFLOP and 1056 B per token-head."""
    b = _bench()
    pm = b.survey_path_model(b.GDN2, dict(B=2, T=4096, H=32, P=64, N=128, C=128))
    assert pm["gdn2"]["fwd"][0] == pytest.approx(95.2e9, rel=2e-3)
    assert pm["gdn2"]["fwd"][1] == pytest.approx(1.21e9, rel=5e-3)
    assert pm["gdn2"]["bwd"][0] == pytest.approx(197.6e9, rel=2e-3)
    assert pm["gdn2"]["bwd"][1] == pytest.approx(2.01e9, rel=5e-3)
    assert pm["mamba2"]["fwd"][0] == pytest.approx(13.2e9, rel=5e-3)
    assert pm["mamba2"]["fwd"][1] == pytest.approx(138e6, rel=5e-3)
    head = b.survey_path_model(b.GDN2, b.MAMBA2)["mamba2"]["fwd"]
    th = b.MAMBA2["B"] * b.MAMBA2["T"] * b.MAMBA2["H"]
    assert head[0] / th == pytest.approx(100.4e3, rel=2e-3)
    assert head[1] / th == pytest.approx(1056)


def test_kernel_shares_cover_the_path_bytes():
    """Every path-level byte lands in some kernel's share: the GDN2 forward
    shares add up to the forward's bytes exactly (o and the inputs are each
    touched by one forward kernel), and every backward output is in a share."""
    b = _bench()
    g, m = b.GDN2, b.MAMBA2
    sh = b.survey_kernel_share(g, m)
    pm = b.survey_path_model(g, m)
    assert sh["gdn2_fwd_intra"] + sh["gdn2_fwd_state"] == pm["gdn2"]["fwd"][1]
    th = g["B"] * g["T"] * g["H"]
    outs = th * (3 * 2 * g["K"] + 2 * 2 * g["V"] + 4 * g["K"])
    assert sh["gdn2_bwd_wy"] + sh["gdn2_bwd_intra"] >= outs
    assert set(sh) == set(b.gdn2_kernel_model(**g)) | set(b.mamba2_kernel_model(**m))
