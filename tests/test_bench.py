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
