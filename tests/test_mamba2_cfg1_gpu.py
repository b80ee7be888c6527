"""Configuration 1 (B2 T4096 H32 P64 N128 C128) on the GPU, fwd + bwd.

At this shape `mamba2_chunk_y` runs its small-grid launch form, 8 (head,
channel slice) pairs per workgroup, so that the grid keeps two workgroups per
CU (larger shapes take 16 pairs, the small test shapes one head's slices);
the state loops run 64-channel heads as two 32-channel workgroups.  Checked
three ways:
  * two heads of the full-shape run against the fp64 oracle (forward: y and
    the final state; backward: ddt, dx, dA, dstate0), and the single-head
    runs' dB / dC against that head's oracle dB / dC;
  * dB / dC of the full shape (summed over the 32 heads in head groups)
    equal to the sum of the 32 single-head runs, whose grids take the
    one-head launch forms.
Reference semantics: mamba2_ssd_reference.py:152-179 and
mamba2_bwd_reference.py:200-266.
"""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import inputs
from atomic_ops import mamba2 as M
from oracle import mamba2 as om

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

BF16 = torch.bfloat16
B1, T1, H1, P1, N1, C1 = 2, 4096, 32, 64, 128, 128
HEADS = (5, 30)


def _errs(pairs):
    out = {n: rel_err(a, b) for n, a, b in pairs}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in out.items()), flush=True)
    return out


def _head(src, j):
    out = {n: src[n][:, :, j:j + 1].contiguous() for n in ("dt", "x", "dy")}
    out.update(Bm=src["Bm"], Cm=src["Cm"], A=src["A"][j:j + 1].contiguous())
    return out


@pytest.fixture(scope="module")
def mamba2_cfg1():
    banner(f"mamba2 cfg1 full shape B{B1} T{T1} H{H1} P{P1} N{N1} C{C1}")
    cpu = inputs.mamba2_inputs(B1, T1, H1, P1, N1, seed=47, dtype=BF16, dO=True)
    dev = {n: t.cuda() for n, t in cpu.items()}
    args = [dev[n] for n in ("dt", "x", "Bm", "Cm", "A")]
    y, sf, ws = M.forward(*args, C1, save=True)
    grads = M.backward(*args, C1, dev["dy"], workspace=ws, reuse=True)
    torch.cuda.synchronize()
    del ws
    return cpu, dev, (y, sf), grads


@pytest.mark.parametrize("j", HEADS)
def test_mamba2_cfg1_head_matches_oracle(mamba2_cfg1, j):
    cpu, dev, (y, sf), grads = mamba2_cfg1
    banner(f"mamba2 cfg1 head {j} against the fp64 oracle")
    hc = _head(cpu, j)
    y_ref, s_ref = om.mamba2_ssd_reference(hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], C1)
    ddt_r, dB_r, dC_r, dx_r, dA_r, ds0_r = om.chunk_ssd_bwd_scan(
        hc["dt"], hc["A"], hc["Bm"], hc["Cm"], hc["x"], C1, hc["dy"])
    ddt, dx, dB, dC, dA, ds0 = grads
    pairs = [("y", y[:, :, j:j + 1], y_ref), ("state", sf[:, j:j + 1], s_ref),
             ("ddt", ddt[:, :, j:j + 1], ddt_r), ("dx", dx[:, :, j:j + 1], dx_r),
             ("dA", dA[j:j + 1], dA_r), ("dstate0", ds0[:, j:j + 1], ds0_r)]
    hd = _head(dev, j)
    g1 = M.backward(*(hd[n] for n in ("dt", "x", "Bm", "Cm", "A")), C1, hd["dy"])
    torch.cuda.synchronize()
    pairs += [("dB(head)", g1[2], dB_r), ("dC(head)", g1[3], dC_r)]
    for n, got, _ in pairs:
        assert torch.isfinite(got.float()).all(), n
    errs = _errs(pairs)
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)


def test_mamba2_cfg1_head_sum_of_dB_dC(mamba2_cfg1):
    _, dev, _, grads = mamba2_cfg1
    banner("mamba2 cfg1 dB / dC head sums")
    sB = torch.zeros_like(dev["Bm"], dtype=torch.float32)
    sC = torch.zeros_like(sB)
    for j in range(H1):
        hd = _head(dev, j)
        g1 = M.backward(*(hd[n] for n in ("dt", "x", "Bm", "Cm", "A")), C1, hd["dy"])
        sB += g1[2].float()
        sC += g1[3].float()
    torch.cuda.synchronize()
    errs = _errs([("dB", grads[2], sB), ("dC", grads[3], sC)])
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)
