"""The epilogue oracle (RMSNorm + SiLU gate, model.py:612-613,650-653 and
:516-525) pinned on the CPU: autograd against central finite differences,
against a hand-derived closed-form VJP, and closed forms of the forward."""
import pytest
import torch

from _util import rel_err
from oracle import norm_gate as ong

F64 = torch.float64
VARIANTS = [ong.GDN2, ong.MAMBA2]


def _inputs(rows, d, seed, gate_scale=3.0, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, d, generator=g, dtype=F64)
    gate = gate_scale * torch.randn(rows, d, generator=g, dtype=F64)
    w = 1.0 + 0.2 * torch.randn(d, generator=g, dtype=F64)
    dout = torch.randn(rows, d, generator=g, dtype=F64)
    return x.to(dtype), gate.to(dtype), w.to(dtype), dout.to(dtype)


@pytest.mark.parametrize("variant", VARIANTS)
def test_autograd_matches_finite_differences(variant):
    x, gate, w, dout = _inputs(3, 8, 0, gate_scale=1.0)
    dx, dg, dw = ong.out_norm_gate_grads(x, gate, w, dout, variant, exact=True)
    h = 1e-6

    def loss(x_, g_, w_):
        return (ong.out_norm_gate(x_, g_, w_, variant, exact=True) * dout).sum()

    for t, grad, which in ((x, dx, 0), (gate, dg, 1), (w, dw, 2)):
        fd = torch.zeros_like(t)
        for idx in range(t.numel()):
            e = torch.zeros_like(t).view(-1)
            e[idx] = h
            e = e.view(t.shape)
            args_p = [x, gate, w]
            args_m = [x, gate, w]
            args_p[which] = t + e
            args_m[which] = t - e
            fd.view(-1)[idx] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        assert rel_err(grad, fd) < 1e-6, which


@pytest.mark.parametrize("variant", VARIANTS)
def test_autograd_matches_closed_form_vjp(variant):
    """dx = d_n w r - x r^3 / d * sum(d_n w x), dweight = sum_rows d_n x r,
    dgate = d_s silu'(g) (masked by the gate clip), r = rsqrt(mean x^2 + eps)."""
    eps = 1e-6
    x, gate, w, dout = _inputs(5, 16, 1, gate_scale=60.0)   # some gates beyond +-100
    dx, dg, dw = ong.out_norm_gate_grads(x, gate, w, dout, variant, eps=eps, exact=True)
    d = x.shape[1]
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    n = x * r * w
    gc = gate.clamp(-1e2, 1e2) if variant == ong.GDN2 else gate
    sg = torch.sigmoid(gc)
    s = gc * sg
    u = dout
    if variant == ong.MAMBA2:
        u = dout * ((n * s).abs() < 3e2)
    dn = u * s
    ds = u * n
    dg_ref = ds * sg * (1 + gc * (1 - sg))
    if variant == ong.GDN2:
        dg_ref = dg_ref * (gate.abs() < 1e2)
    dx_ref = dn * w * r - x * r ** 3 / d * (dn * w * x).sum(-1, keepdim=True)
    dw_ref = (dn * x * r).sum(0)
    assert rel_err(dx, dx_ref) < 1e-12
    assert rel_err(dg, dg_ref) < 1e-12
    assert rel_err(dw, dw_ref) < 1e-12


@pytest.mark.parametrize("variant", VARIANTS)
def test_forward_closed_forms(variant):
    x, gate, w, _ = _inputs(4, 32, 2)
    # unit weight: the normalised rows have mean square ms / (ms + eps)
    eps = 1e-6
    n = ong.rms_norm(x, torch.ones(32, dtype=F64), eps)
    ms = (x * x).mean(-1)
    assert rel_err((n * n).mean(-1), ms / (ms + eps)) < 1e-12
    # a zero gate zeroes the output and every gradient but the gate's
    z = torch.zeros_like(gate)
    out = ong.out_norm_gate(x, z, w, variant, exact=True)
    assert out.abs().max() == 0
    dx, dg, dw = ong.out_norm_gate_grads(x, z, w, torch.ones_like(x), variant, exact=True)
    assert dx.abs().max() == 0 and dw.abs().max() == 0
    # silu'(0) = 1/2: dgate = n / 2
    n_full = ong.rms_norm(x, w, eps)
    assert rel_err(dg, 0.5 * n_full) < 1e-12


def test_gdn2_gate_clip_bound_and_tie():
    x, _, w, _ = _inputs(2, 8, 3)
    gate = torch.full((2, 8), 250.0, dtype=F64)
    gate[0, 0] = 100.0
    gate[1, 1] = -100.0
    out = ong.out_norm_gate(x, gate, w, ong.GDN2, exact=True)
    n = ong.rms_norm(x, w, 1e-6)
    gc = torch.full((2, 8), 100.0, dtype=F64)       # 250 and 100 both enter as 100
    gc[1, 1] = -100.0
    assert rel_err(out, n * torch.nn.functional.silu(gc)) < 1e-12
    _, dg, _ = ong.out_norm_gate_grads(x, gate, w, torch.ones_like(x), ong.GDN2, exact=True)
    mask = torch.zeros(2, 8, dtype=F64)
    mask[0, 0] = 0.5                                # ties split the cotangent
    expect = n * torch.sigmoid(gate.clamp(-1e2, 1e2)) * (1 + gate.clamp(-1e2, 1e2) *
                                                          (1 - torch.sigmoid(gate.clamp(-1e2, 1e2))))
    assert rel_err(dg, expect * mask) < 1e-12
    assert dg[1, 1] == 0 or abs(dg[1, 1].item()) < 1e-30   # silu'(-100) underflows to ~0


@pytest.mark.parametrize("variant", VARIANTS)
def test_bf16_flow_stays_near_exact(variant):
    x, gate, w, dout = _inputs(16, 512, 4, dtype=torch.float32)
    gate_b = gate.to(torch.bfloat16)
    ref = ong.out_norm_gate(x.double(), gate_b.double(), w.double(), variant, exact=True)
    out = ong.out_norm_gate(x, gate_b, w, variant)
    assert out.dtype == torch.bfloat16
    assert rel_err(out, ref) < 2e-2
