"""Fused output epilogue (RMSNorm + SiLU gate) on the GPU, through the C ABI,
against the CPU oracle's bf16 dtype flow (model.py:612-613,650-653 for GDN2,
:516-525 for Mamba2).  Tolerance: the bf16 north-star bound, 2e-2."""
import pytest
import torch

from _util import TOL_BF16, banner, rel_err
from atomic_ops import _lib
from atomic_ops import norm_gate as NG
from oracle import norm_gate as ong

pytestmark = pytest.mark.gpu

VARIANTS = [(NG.GDN2, ong.GDN2), (NG.MAMBA2, ong.MAMBA2)]


def _inputs(rows, d, seed, gate_scale):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, d, generator=g)
    gate = (gate_scale * torch.randn(rows, d, generator=g)).to(torch.bfloat16)
    w = 1.0 + 0.2 * torch.randn(d, generator=g)
    dout = torch.randn(rows, d, generator=g).to(torch.bfloat16)
    return x, gate, w, dout


@pytest.mark.parametrize("variant,ovar", VARIANTS)
@pytest.mark.parametrize("rows,d,gate_scale", [
    (37, 512, 3.0),      # ragged row count (last workgroup partly idle)
    (256, 2048, 3.0),    # the benchmark's model dimension (H 16 x 128)
    (64, 1536, 60.0),    # three pieces per lane; gates beyond the +-1e2 clip
    (9, 8192, 3.0),      # the largest supported dimension (a workgroup per row in the backward)
    (1100, 4096, 3.0),   # the smallest workgroup-per-row width; rows beyond the 512 partial rows
    (13, 6144, 60.0),    # twelve pieces per row: three per wave
    (300, 1024, 3.0),    # two pieces per lane
    (129, 3072, 60.0),   # six pieces per lane, one row past a workgroup of four
])
def test_epilogue_matches_oracle(variant, ovar, rows, d, gate_scale):
    banner(f"norm_gate {ovar} rows={rows} d={d} gate_scale={gate_scale}")
    x, gate, w, dout = _inputs(rows, d, rows + d, gate_scale)
    if ovar == ong.MAMBA2:
        x = x * 40.0          # products beyond the +-3e2 clip
    out_ref = ong.out_norm_gate(x, gate, w, ovar)
    dx_ref, dg_ref, dw_ref = ong.out_norm_gate_grads(x, gate, w, dout, ovar)
    xc, gc, wc = x.cuda(), gate.cuda(), w.cuda()
    out = NG.forward(xc, gc, wc, variant)
    dx, dg, dw = NG.backward(xc, gc, wc, dout.cuda(), variant)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and dg.dtype == torch.bfloat16
    assert dx.dtype == torch.float32 and dw.dtype == torch.float32
    for name, a, b in (("out", out, out_ref), ("dx", dx, dx_ref), ("dgate", dg, dg_ref), ("dweight", dw, dw_ref)):
        e = rel_err(a, b)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name


def test_autograd_wrapper_and_shapes():
    banner("norm_gate autograd wrapper, [B, T, H, V] input")
    B, T, H, V = 2, 48, 4, 128
    g = torch.Generator().manual_seed(7)
    o = torch.randn(B, T, H, V, generator=g)
    gate = torch.randn(B, T, H * V, generator=g).to(torch.bfloat16)
    w = 1.0 + 0.1 * torch.randn(H * V, generator=g)
    dout = torch.randn(B, T, H * V, generator=g).to(torch.bfloat16)
    oc = o.cuda().requires_grad_(True)
    gc = gate.cuda().requires_grad_(True)
    wc = w.cuda().requires_grad_(True)
    out = NG.gdn2_out_norm_gate(oc, gc, wc)
    out.backward(dout.cuda())
    ref = ong.out_norm_gate(o.view(B * T, H * V), gate.view(B * T, H * V), w, ong.GDN2)
    dx_ref, dg_ref, dw_ref = ong.out_norm_gate_grads(o.view(B * T, H * V), gate.view(B * T, H * V), w,
                                                     dout.view(B * T, H * V), ong.GDN2)
    assert out.shape == gate.shape and oc.grad.shape == o.shape
    assert rel_err(out.view(B * T, -1), ref) < TOL_BF16
    assert rel_err(oc.grad.view(B * T, -1), dx_ref) < TOL_BF16
    assert rel_err(gc.grad.view(B * T, -1), dg_ref) < TOL_BF16
    assert rel_err(wc.grad, dw_ref) < TOL_BF16


def test_unsupported_dimension_is_rejected_before_launch():
    banner("norm_gate shape error")
    x = torch.zeros(4, 640, device="cuda")
    gate = torch.zeros(4, 640, dtype=torch.bfloat16, device="cuda")
    w = torch.ones(640, device="cuda")
    with pytest.raises(_lib.AtomicError, match="SHAPE"):
        NG.forward(x, gate, w, NG.GDN2)
