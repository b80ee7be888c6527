"""Mamba2 with float32 operands, on the GPU.

The reference's Mamba2 stages take dt, x, B, C in whatever dtype the model
runs in and upcast to float32 (kernel_mamba2_a_decay.py:80-82,
kernel_mamba2_b_intra.py:31-36, kernel_mamba2_bwd_b1_state.py:168-172).  With
float32 operands the library runs its float32 staged chain at the caller's
chunk: M2 -> M3 -> M4 forward (kernel_mamba2_c_interchunk.py:90-100) and
MB1 + MB3 -> MB4 backward, composed as the trainable op does
(kernel_mamba2_trainable_B6.py:72-131).  The forward is compared with the
oracle's staged composition and with the chunked reference
(mamba2_ssd_reference.py:152-179; every step exponent dt A < 0 here, where the
two agree), the backward with the oracle's MB0 (mamba2_bwd_reference.py:55-266)
after the trainable op's final clip.  Float32 operands: float32 tolerance.
"""
import ctypes

import pytest
import torch

from _util import TOL_F32, banner, rel_err
from atomic_ops import _lib
from atomic_ops import inputs
from atomic_ops import kernel_mamba2_a_decay as MA
from atomic_ops import kernel_mamba2_b_intra as MBI
from atomic_ops import kernel_mamba2_bwd_b1_state as MB1
from atomic_ops import kernel_mamba2_bwd_b2_intra as MB2
from atomic_ops import kernel_mamba2_c_interchunk as MC
from atomic_ops import kernel_mamba2_trainable_B6 as T6
from atomic_ops import mamba2 as M
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

F32 = torch.float32


def _check(name, got, ref, tol=TOL_F32):
    e = rel_err(got, ref)
    print(f"  {name}: rel_err {e:.2e}", flush=True)
    assert tuple(got.shape) == tuple(ref.shape) and got.dtype == F32 and e < tol, (name, e)


def _inputs(b, l, h, P, N, seed):
    d = inputs.mamba2_inputs(b, l, h, P, N, seed=seed, dtype=F32, dO=True)
    dt, x, Bm, Cm, A, dy = (d[n] for n in ("dt", "x", "Bm", "Cm", "A", "dy"))
    gen = torch.Generator().manual_seed(seed + 1)
    dsf = 0.3 * torch.randn(b, h, P, N, generator=gen)
    s0 = 0.3 * torch.randn(b, h, P, N, generator=gen)
    return dt, x, Bm, Cm, A, dy, dsf, s0


def _mb0_order(mb0):
    """MB0 returns (ddt, dB, dC, dx, dA, dstate0); the op's order is the primals'."""
    ddt, dB, dC, dx, dA, ds0 = mb0
    return ddt, dx, dB, dC, dA, ds0


CASES = [(64, 2, 512, 2, 64, 128), (128, 1, 512, 3, 128, 64), (256, 1, 768, 2, 64, 128),
         (256, 1, 512, 2, 192, 128),
         # a state size above heads x channels (N > H P): the dC / dB arrays are
         # the longest of the backward's final element-wise pass
         (128, 2, 512, 1, 64, 128), (256, 2, 512, 1, 64, 128)]


@pytest.mark.parametrize("C,b,l,h,P,N", CASES)
def test_mamba2_f32_stages_match_the_oracle(C, b, l, h, P, N):
    """M2, M3, M4 alone and chained, float32 operands, at each chunk."""
    banner(f"mamba2 f32 stages chunk {C} B{b} T{l} H{h} P{P} N{N}")
    dt, x, Bm, Cm, A, _, _, s0 = _inputs(b, l, h, P, N, 600 + C + P)
    cum_r = om.build_chunk_cumdecay(dt, A, C)
    yd_r, se_r = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_r, C)
    y_r, sf_r = om.mamba2_inter_chunk_combine(yd_r, se_r, cum_r, Cm, C, state0=s0)
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    cum = MA.build_chunk_cumdecay_pallas(g[0], g[4], C)
    yd, se = MBI.intra_chunk_ssd_pallas(g[0], g[1], g[2], g[3], cum_r.float().cuda(), C)
    y, sf = MC.mamba2_inter_chunk_combine(yd_r.float().cuda(), se_r.float().cuda(), cum_r.float().cuda(), g[3], C,
                                          state0=s0.cuda())
    ys, sfs = MC.mamba2_pallas_forward(*g, C, state0=s0.cuda())
    torch.cuda.synchronize()
    _check("cumdecay", cum, cum_r)
    _check("y_diag", yd, yd_r)
    _check("state_end", se, se_r)
    _check("y", y, y_r)
    _check("state_final", sf, sf_r)
    _check("staged y", ys, y_r)
    _check("staged state_final", sfs, sf_r)


@pytest.mark.parametrize("C,b,l,h,P,N", CASES)
def test_mamba2_f32_whole_path_matches_the_oracle(C, b, l, h, P, N):
    """atomic_mamba2_fwd / atomic_mamba2_bwd with float32 operands: forward
    against the staged oracle and the chunked reference, gradients (float32,
    the primals' dtype) against MB0 after the final clip."""
    banner(f"mamba2 f32 whole path chunk {C} B{b} T{l} H{h} P{P} N{N}")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _inputs(b, l, h, P, N, 700 + C + P)
    cum_r = om.build_chunk_cumdecay(dt, A, C)
    yd_r, se_r = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_r, C)
    y_r, sf_r = om.mamba2_inter_chunk_combine(yd_r, se_r, cum_r, Cm, C, state0=s0)
    y_c, sf_c = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0)
    mb0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    y, sf, ws = M.forward(*g, C, state0=s0.cuda())
    grads = M.backward(*g, C, dy.cuda(), dsf.cuda(), state0=s0.cuda(), workspace=ws)
    torch.cuda.synchronize()
    _check("y (staged)", y, y_r)
    _check("state_final (staged)", sf, sf_r)
    _check("y (chunked reference)", y, y_c)
    _check("state_final (chunked reference)", sf, sf_c)
    for n, g_, r in zip(("ddt", "dx", "dB", "dC", "dA", "dstate0"), grads, _mb0_order(mb0)):
        _check(f"MB0 {n}", g_, om.final_sanitize(r))


def test_mamba2_f32_trainable_op_matches_mb0():
    """The drop-in trainable op on float32 leaves: autograd's gradients, in
    float32, against MB0 after the final clip."""
    C, b, l, h, P, N = 128, 2, 512, 2, 64, 128
    banner("mamba2 f32 trainable op")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _inputs(b, l, h, P, N, 801)
    mb0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    leaves = [t.cuda().requires_grad_() for t in (dt, x, Bm, Cm, A, s0)]
    y, sf = T6.mamba2_pallas_forward_trainable_B6(*leaves[:5], C, state0=leaves[5])
    torch.autograd.backward((y, sf), (dy.cuda(), dsf.cuda()))
    torch.cuda.synchronize()
    y_c, _ = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0)
    _check("y", y.detach(), y_c)
    for n, leaf, r in zip(("ddt", "dx", "dB", "dC", "dA", "dstate0"), leaves, _mb0_order(mb0)):
        _check(f"grad {n}", leaf.grad, om.final_sanitize(r))


@pytest.mark.parametrize("C", [64, 256])
def test_mamba2_f32_backward_stages_match_the_oracle(C):
    """MB2 and MB1 + MB3 on float32 operands against the oracle."""
    b, l, h, P, N = 1, 512, 2, 128, 64
    banner(f"mamba2 f32 MB1 / MB2 chunk {C}")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _inputs(b, l, h, P, N, 900 + C)
    gen = torch.Generator().manual_seed(901 + C)
    dse = 0.3 * torch.randn(b, h, l // C, P, N, generator=gen)
    cum = om.build_chunk_cumdecay(dt, A, C).float()
    ref2 = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum.double(), dy.double(), dse.double(), C)
    got2 = MB2.intra_chunk_ssd_bwd_pallas(dt.cuda(), x.cuda(), Bm.cuda(), Cm.cuda(), cum.cuda(), dy.cuda(),
                                          dse.cuda(), C)
    ref1 = om.mamba2_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    got1 = MB1.mamba2_bwd_scan(dt.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), x.cuda(), C, dy.cuda(), dsf.cuda(),
                               state0=s0.cuda())
    torch.cuda.synchronize()
    for n, g_, r in zip(("ddt", "dx", "dB", "dC", "dcum"), got2, ref2):
        _check(f"MB2 {n}", g_, r)
    for n, g_, r in zip(("ddt", "dB", "dC", "dx", "dstate0", "dcumdecay"), got1, ref1):
        _check(f"MB1+MB3 {n}", g_, r)


def test_mamba2_f32_rejects_stage_reports():
    """Stage reports cover the bf16 whole-path kernels only: a float32 call
    that asks for them is refused before any launch."""
    banner("mamba2 f32 diag refused")
    dt, x, Bm, Cm, A, _, _, _ = _inputs(1, 256, 2, 64, 64, 950)
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    reports = _lib.StageReports(_lib.MAMBA2_DIAG_STAGES, torch.device("cuda"))
    with pytest.raises(_lib.AtomicError):
        M.forward(*g, 128, diag=reports)
    args = M.make_args(g[0], g[2], 128)
    assert _lib.load().atomic_mamba2_workspace_size(ctypes.byref(args)) > 0


def test_mamba2_f32_backward_without_dstate0():
    """dstate0 may be NULL (atomic_mamba2_bwd): the float32 chain then keeps
    it in the workspace, and every other gradient is bit-identical to the
    call that asks for it."""
    C, b, l, h, P, N = 128, 1, 512, 2, 64, 128
    banner("mamba2 f32 backward, dstate0 NULL")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _inputs(b, l, h, P, N, 960)
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    ref = M.backward(*g, C, dy.cuda(), dsf.cuda(), state0=s0.cuda())
    args = M.make_args(g[0], g[2], C, dy_dtype=F32)
    lib = _lib.load()
    ws = torch.empty(lib.atomic_mamba2_workspace_size(ctypes.byref(args)), dtype=torch.uint8, device="cuda")
    out = [torch.empty_like(t) for t in (g[0], g[1], g[2], g[3])] + [torch.empty(h, device="cuda")]
    p = M._ptr
    dyc, dsfc, s0c = dy.cuda(), dsf.cuda(), s0.cuda()
    rc = lib.atomic_mamba2_bwd(ctypes.byref(args), *(p(t) for t in g), p(s0c), p(dyc), p(dsfc),
                               *(p(t) for t in out), p(None), p(ws), ctypes.c_size_t(ws.numel()),
                               M._stream(g[0].device))
    _lib.check(rc, "atomic_mamba2_bwd")
    torch.cuda.synchronize()
    for n, a_, r in zip(("ddt", "dx", "dB", "dC", "dA"), out, ref[:5]):
        assert torch.equal(a_, r), n


def test_mamba2_f32_positive_exponent_follows_the_stage_kernels():
    """A head with A > 0 (every step exponent dt A positive), where the
    reference's stage kernels and mamba2_ssd_reference part ways (no 1e6
    caps in the former), and a head with A = -200 (step exponents past the
    -20 clip, so M2's and MB4's clip masks act): the float32 whole path
    follows the staged chain, forward against the oracle's M2 -> M3 -> M4
    and backward against the oracle's MB1 + MB3 and MB4 composed as the
    trainable op."""
    from atomic_ops import mamba2_bwd_a_dA_reference as MB4
    C, b, l, h, P, N = 64, 1, 256, 2, 64, 64
    banner("mamba2 f32 positive step exponent")
    dt, x, Bm, Cm, A, dy, dsf, s0 = _inputs(b, l, h, P, N, 970)
    A = A.clone()
    A[0], A[1] = 0.05, -200.0
    cum_r = om.build_chunk_cumdecay(dt, A, C)
    assert (cum_r[:, 0] > 0).any(), "the exponent must be positive"
    assert ((dt[..., 1, :].double() * A[1]) < -20).any(), "some steps must pass the clip"
    yd_r, se_r = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_r, C)
    y_r, sf_r = om.mamba2_inter_chunk_combine(yd_r, se_r, cum_r, Cm, C, state0=s0)
    sc = om.mamba2_bwd_scan(dt, A, Bm, Cm, x, C, dy.double(), dsf.double(), s0.double())
    ddt2, dA_r = om.mamba2_dA_backward(MB4.reshape_dt_to_pallas(dt, C), A, sc[5], C)
    fin = om.final_sanitize
    ref = (fin(sc[0] + MB4.unreshape_dt_from_pallas(ddt2)), fin(sc[3]), fin(sc[1]), fin(sc[2]), fin(dA_r), fin(sc[4]))
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    y, sf, ws = M.forward(*g, C, state0=s0.cuda())
    grads = M.backward(*g, C, dy.cuda(), dsf.cuda(), state0=s0.cuda(), workspace=ws)
    torch.cuda.synchronize()
    _check("y", y, y_r)
    _check("state_final", sf, sf_r)
    for n, g_, r in zip(("ddt", "dx", "dB", "dC", "dA", "dstate0"), grads, ref):
        _check(f"staged {n}", g_, r)
