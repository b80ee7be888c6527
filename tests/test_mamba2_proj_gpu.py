"""Mamba2 prologue with its projections (model.py:405-433) on the GPU, through
the C ABI: the in_proj output read in place (x_bc = its first d_inner columns),
the dt / B / C projections as one MFMA GEMM with the activation epilogue, and
the backward's dX / dW GEMMs, against the CPU oracle's bf16 dtype flow.
Tolerance: the bf16 north-star bound, 2e-2 (norm-wise per tensor)."""
import pytest
import torch

from _util import TOL_BF16, banner, rel_err
from atomic_ops import _lib
from atomic_ops import prologue as PL
from oracle import prologue as op

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
OUTS = ("x", "dt", "B", "C", "A")
PRES = ("dt_pre", "b_pre", "c_pre")
GRADS = ("dx_bc", "dconv_w", "dconv_b", "dw_dt", "db_dt", "dw_b", "dw_c", "da_log")


def _inputs(B, L, H, P, N, seed):
    """(in_proj [B, L, 2 d] bf16, params...) and the cotangents of (x, dt, B, C, A)."""
    g = torch.Generator().manual_seed(seed)
    d = H * P
    r = lambda *s: torch.randn(*s, generator=g)
    in_proj = r(B, L, 2 * d).to(BF16)
    params = [0.5 * r(d, 4), 0.1 * r(d), r(d, d) / d ** 0.5, r(d) - 2.0, r(d, N) / d ** 0.5, r(d, N) / d ** 0.5,
              r(H)]
    cots = [r(B, L, H, P).to(BF16), r(B, L, H, P).to(BF16), r(B, L, N).to(BF16), r(B, L, N).to(BF16), r(H)]
    return in_proj, params, cots


def _check(names, got, ref):
    for name, a, b in zip(names, got, ref):
        assert a.dtype == b.dtype and a.shape == b.shape, (name, a.dtype, b.dtype, a.shape, b.shape)
        e = rel_err(a, b)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name


@pytest.mark.parametrize("B,L,H,P,N", [
    (2, 128, 4, 128, 64),     # two sequences, d_inner 512, N 64
    (1, 256, 8, 64, 128),     # headdim 64
    (1, 256, 16, 128, 128),   # the benchmark's Mamba2 head shape (d_inner 2048)
])
def test_proj_prologue_matches_oracle(B, L, H, P, N):
    banner(f"mamba2 proj prologue B={B} L={L} H={H} P={P} N={N}")
    in_proj, params, cots = _inputs(B, L, H, P, N, 31 * B + L + H + P + N)
    d = H * P
    x_bc = in_proj[..., :d]                          # jnp.split's first half (model.py:406)
    ref_out = op.mamba2_proj_prologue(x_bc, *params, H)
    ref_pre = op.mamba2_projections(x_bc, *params[2:6])
    ref_grads = op.mamba2_proj_prologue_grads([x_bc] + params, cots, H)

    gp = in_proj.cuda()
    gparams = [t.cuda() for t in params]
    outs, pres = PL.mamba2_proj_forward(gp[..., :d], *gparams, H, save=True)
    # the gradient lands in the x_bc half of the in_proj gradient; the other half is left alone
    d_in = torch.full_like(gp, 7.0)
    grads = PL.mamba2_proj_backward(gp[..., :d], *gparams, H, pres, *(c.cuda() for c in cots), dx_bc=d_in)
    torch.cuda.synchronize()
    _check(OUTS, outs, ref_out)
    _check(PRES, pres, ref_pre)
    _check(GRADS, grads, ref_grads)
    assert torch.equal(d_in[..., d:].cpu(), torch.full((B, L, d), 7.0, dtype=BF16))
    assert grads[0].data_ptr() == d_in.data_ptr()


def test_whole_in_proj_tensor_and_autograd_wrapper():
    """Mamba2ProjPrologue over the whole in_proj output: the x_bc half's gradient
    equals the direct call's, the res half's is zero, parameters' grads match."""
    banner("mamba2 proj prologue autograd wrapper")
    B, L, H, P, N = 1, 128, 4, 128, 64
    in_proj, params, cots = _inputs(B, L, H, P, N, 5)
    d = H * P
    gp = in_proj.cuda().requires_grad_(True)
    gparams = [t.cuda().requires_grad_(True) for t in params]
    outs = PL.Mamba2ProjPrologue.apply(gp, *gparams, H)
    torch.autograd.backward(outs, [c.cuda() for c in cots])
    ref_grads = op.mamba2_proj_prologue_grads([in_proj[..., :d]] + params, cots, H)
    assert rel_err(gp.grad[..., :d], ref_grads[0]) < TOL_BF16
    assert torch.count_nonzero(gp.grad[..., d:]).item() == 0
    for name, leaf, r in zip(GRADS[1:], gparams, ref_grads[1:]):
        e = rel_err(leaf.grad, r)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name


def test_fused_equals_unfused_prologue():
    """The fused forward against the element-wise prologue entry fed with the
    projection outputs the fused call saved: x, dt, B, C, A bit-identical."""
    banner("mamba2 proj prologue vs element-wise entry")
    B, L, H, P, N = 1, 128, 8, 64, 64
    in_proj, params, _ = _inputs(B, L, H, P, N, 9)
    d = H * P
    gp = in_proj.cuda()
    gparams = [t.cuda() for t in params]
    outs, (dt_pre, b_pre, c_pre) = PL.mamba2_proj_forward(gp[..., :d], *gparams, H, save=True)
    ref = PL.mamba2_forward(gp[..., :d].contiguous(), gparams[0], gparams[1], dt_pre, b_pre, c_pre, gparams[6], H)
    for name, a, b in zip(OUTS, outs, ref):
        assert torch.equal(a, b), name


def test_unsupported_shapes_are_rejected_before_launch():
    banner("mamba2 proj prologue shape errors")
    in_proj, params, _ = _inputs(1, 128, 4, 128, 32, 3)   # N = 32: not a multiple of 64
    gparams = [t.cuda() for t in params]
    with pytest.raises(_lib.AtomicError, match="unsupported shape"):
        PL.mamba2_proj_forward(in_proj.cuda()[..., :512], *gparams, 4)
