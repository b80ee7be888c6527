"""Fused GDN2 prologue (model.py:574-619) on the GPU, through the C ABI,
against the CPU oracle's bf16 dtype flow.  Tolerance: the bf16 north-star
bound, 2e-2 (norm-wise per tensor)."""
import pytest
import torch

from _util import TOL_BF16, banner, rel_err
from atomic_ops import _lib
from atomic_ops import prologue as PL
from oracle import prologue as op

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
OUT_NAMES = ("q", "k", "v", "w", "b", "g")
GRAD_NAMES = ("dq_lin", "dk_lin", "dv_lin", "dconv_w", "dconv_b", "db_pre", "dw_pre", "df_pre", "da")


def _inputs(B, L, H, dh, seed):
    g = torch.Generator().manual_seed(seed)
    d = H * dh
    r = lambda *s: torch.randn(*s, generator=g)
    ins = [r(B, L, d).to(BF16) for _ in range(3)] + [0.5 * r(3, d, 4), 0.1 * r(3, d)]
    ins += [r(B, L, d).to(BF16), r(B, L, d).to(BF16), (r(B, L, d) + 1.0).to(BF16), r(H)]
    cots = [r(B, L, H, dh).to(BF16) for _ in range(5)] + [r(B, L, H, dh)]
    return ins, cots


@pytest.mark.parametrize("B,L,H,dh", [
    (2, 128, 4, 128),     # d = 512, two sequences (the conv restarts at each)
    (1, 256, 8, 64),      # dh = 64: eight lanes per head
    (1, 128, 16, 128),    # the benchmark's d = 2048
])
def test_prologue_matches_oracle(B, L, H, dh):
    banner(f"prologue B={B} L={L} H={H} dh={dh}")
    ins, cots = _inputs(B, L, H, dh, B * 1000 + L + H + dh)
    ref_out = op.gdn2_prologue(*ins, H)
    ref_grads = op.gdn2_prologue_grads(ins, cots, H)
    gi = [t.cuda() for t in ins]
    outs = PL.forward(*gi, H)
    grads = PL.backward(*gi, H, *(c.cuda() for c in cots))
    torch.cuda.synchronize()
    for name, a, b in zip(OUT_NAMES, outs, ref_out):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        e = rel_err(a, b)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name
    for name, a, b in zip(GRAD_NAMES, grads, ref_grads):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        e = rel_err(a, b)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name


def test_autograd_wrapper():
    banner("prologue autograd wrapper")
    B, L, H, dh = 1, 128, 4, 128
    ins, cots = _inputs(B, L, H, dh, 11)
    leaves = [t.cuda().requires_grad_(t.is_floating_point()) for t in ins]
    outs = PL.GDN2Prologue.apply(*leaves, H)
    torch.autograd.backward(outs, [c.cuda() for c in cots])
    ref = op.gdn2_prologue_grads(ins, cots, H)
    for name, leaf, r in zip(GRAD_NAMES, leaves, ref):
        assert rel_err(leaf.grad, r) < TOL_BF16, name


def test_unsupported_shape_is_rejected_before_launch():
    banner("prologue shape error")
    ins, _ = _inputs(1, 96, 4, 128, 3)      # L not a multiple of 128
    with pytest.raises(_lib.AtomicError, match="SHAPE"):
        PL.forward(*(t.cuda() for t in ins), 4)


M2_OUT = ("x", "dt", "B", "C", "A")
M2_GRADS = ("dx_bc", "dconv_w", "dconv_b", "ddt_pre", "db_pre", "dc_pre", "da_log")


def _m2_inputs(B, L, H, P, N, seed):
    g = torch.Generator().manual_seed(seed)
    d = H * P
    r = lambda *s: torch.randn(*s, generator=g)
    ins = [r(B, L, d).to(BF16), 0.5 * r(d, 4), 0.1 * r(d), (2.0 * r(B, L, d) - 1.0).to(BF16),
           r(B, L, N).to(BF16), r(B, L, N).to(BF16), r(H)]
    cots = [r(B, L, H, P).to(BF16), r(B, L, H, P).to(BF16), r(B, L, N).to(BF16), r(B, L, N).to(BF16), r(H)]
    return ins, cots


@pytest.mark.parametrize("B,L,H,P,N", [
    (2, 128, 4, 128, 64),     # two sequences, d_inner 512
    (1, 256, 16, 128, 128),   # the benchmark's Mamba2 head shape (d_inner 2048)
])
def test_mamba2_prologue_matches_oracle(B, L, H, P, N):
    banner(f"mamba2 prologue B={B} L={L} H={H} P={P} N={N}")
    ins, cots = _m2_inputs(B, L, H, P, N, B + L + H + N)
    ref_out = op.mamba2_prologue(*ins, H)
    ref_grads = op.mamba2_prologue_grads(ins, cots, H)
    gi = [t.cuda() for t in ins]
    outs = PL.mamba2_forward(*gi, H)
    grads = PL.mamba2_backward(*gi, H, *(c.cuda() for c in cots))
    torch.cuda.synchronize()
    for name, a, b in list(zip(M2_OUT, outs, ref_out)) + list(zip(M2_GRADS, grads, ref_grads)):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        e = rel_err(a, b)
        print(f"  {name}: rel_err {e:.2e}")
        assert e < TOL_BF16, name
