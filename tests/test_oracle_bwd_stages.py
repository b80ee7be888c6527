"""Pins the oracle's backward stage restatements at the reference's 256-row block.

* GDN2 kernels B2, B1, B3, B4, B5 (kernel_bwd_b2_dav.py, kernel_bwd_b1_dhu.py,
  kernel_bwd_b3_wy_dqkg.py, kernel_bwd_b4_intra.py,
  kernel_bwd_b5_reverse_cumsum.py), composed as the reference's trainable op
  composes them (kernel_trainable_B6.py:97-181), give the gradient of the
  chunked reference at chunk 256 that torch autograd computes
  (gdn2_backward_autodiff, itself pinned by finite differences).
* Mamba2 MB2 (kernel_mamba2_bwd_b2_intra.py:32-180) is the vector-Jacobian
  product of M3 (intra_chunk_ssd, pinned by the element-by-element loops):
  the same cotangents through torch autograd give the same five gradients.
* Mamba2 MB1 + MB3 (mamba2_bwd_scan, kernel_mamba2_bwd_b1_state.py:132-254)
  and MB4 (mamba2_dA_backward, mamba2_bwd_a_dA_reference.py:60-115), composed
  as the trainable op composes them (kernel_mamba2_trainable_B6.py:83-131),
  equal MB0's per-chunk backward (pinned against autograd).
* Planted mistakes in a stage fail the composition.
"""
import torch

from oracle import gdn2 as og
from oracle import mamba2 as om

F64 = torch.float64


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def _gdn2_case(seed=21, T=512, H=2, K=16, V=12):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(1, T, H, K, generator=gen, dtype=F64)
    k = torch.randn(1, T, H, K, generator=gen, dtype=F64)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(1, T, H, V, generator=gen, dtype=F64)
    b = torch.sigmoid(torch.randn(1, T, H, K, generator=gen, dtype=F64))
    w = torch.sigmoid(torch.randn(1, T, H, V, generator=gen, dtype=F64))
    g = torch.nn.functional.logsigmoid(3.0 + torch.randn(1, T, H, K, generator=gen, dtype=F64))
    do = torch.randn(1, T, H, V, generator=gen, dtype=F64)
    dhf = 0.3 * torch.randn(1, H, K, V, generator=gen, dtype=F64)
    h0 = 0.3 * torch.randn(1, H, K, V, generator=gen, dtype=F64)
    return q, k, v, w, b, g, do, dhf, h0


def test_gdn2_backward_stages_compose_to_autodiff():
    q, k, v, w, b, g, do, dhf, h0 = _gdn2_case()
    got = og.gdn2_backward_staged(q, k, v, w, b, g, 0.7, do, dh_final=dhf, h0=h0)
    ref = og.gdn2_backward_autodiff(q, k, v, w, b, g, 0.7, 256, do, dh_final=dhf, h0=h0)
    for name, a, c in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), got, ref):
        assert _rel(a, c) < 1e-11, name


def test_gdn2_backward_stage_mistakes_are_caught(monkeypatch):
    q, k, v, w, b, g, do, dhf, h0 = _gdn2_case(seed=4)
    ref = og.gdn2_backward_autodiff(q, k, v, w, b, g, 0.7, 256, do, dh_final=dhf, h0=h0)

    def worst(got):
        return max(_rel(a, c) for a, c in zip(got, ref))

    # (1) B1 without the decay of the carried gradient
    real_dhu = og.dhu_backward

    def no_decay(do_, dvp, wp, qg, kg, gcl, scale, dht=None, dtype=F64):
        return real_dhu(do_, dvp, wp, qg, kg, torch.zeros_like(gcl), scale, dht=dht, dtype=dtype)
    monkeypatch.setattr(og, "dhu_backward", no_decay)
    assert worst(og.gdn2_backward_staged(q, k, v, w, b, g, 0.7, do, dh_final=dhf, h0=h0)) > 1e-6
    monkeypatch.undo()

    # (2) B3 without the gc_last row term of the state decay
    real_b3 = og.wy_dqkg_backward

    def no_row_term(q_, k_, b_, w_, v_, gc, A, Akk, h_pre, v_new, do_, dv, dh_next, scale, dtype=F64):
        return real_b3(q_, k_, b_, w_, v_, gc, A, Akk, h_pre, v_new, do_, dv, torch.zeros_like(dh_next),
                       scale, dtype=dtype)
    monkeypatch.setattr(og, "wy_dqkg_backward", no_row_term)
    assert worst(og.gdn2_backward_staged(q, k, v, w, b, g, 0.7, do, dh_final=dhf, h0=h0)) > 1e-6
    monkeypatch.undo()

    # (3) B4 with dAqk transposed
    real_b4 = og.intra_backward

    def transposed(dAqk, dAkk, *a, **kw):
        return real_b4(dAqk.transpose(-1, -2).tril(), dAkk, *a, **kw)
    monkeypatch.setattr(og, "intra_backward", transposed)
    assert worst(og.gdn2_backward_staged(q, k, v, w, b, g, 0.7, do, dh_final=dhf, h0=h0)) > 1e-6


def test_gdn2_b4_clips_every_accumulation():
    """With dAqk so large that single sub-block pair sums pass the clip,
    every output stays within +-1e4 and finite (kernel_bwd_b4_intra.py:113-121)."""
    q, k, v, w, b, g, do, dhf, h0 = _gdn2_case(seed=8)
    dAqk = 1e9 * torch.randn(1, 2, 2, 256, 256, dtype=F64)
    dAkk = -1e9 * torch.randn(1, 2, 2, 256, 256, dtype=F64)
    for t in og.intra_backward(dAqk, dAkk, q, k, b, g, 0.7):
        assert torch.isfinite(t).all() and t.abs().max().item() <= 1e4


def _mamba2_case(seed=3, l=512, h=2, p=8, n=6, C=256):
    gen = torch.Generator().manual_seed(seed)
    dt = torch.nn.functional.softplus(torch.randn(1, l, h, p, generator=gen, dtype=F64) - 3)
    x = torch.randn(1, l, h, p, generator=gen, dtype=F64)
    Bm = torch.randn(1, l, n, generator=gen, dtype=F64) / n ** 0.5
    Cm = torch.randn(1, l, n, generator=gen, dtype=F64) / n ** 0.5
    A = -0.5 * torch.rand(h, generator=gen, dtype=F64)
    cum = om.build_chunk_cumdecay(dt, A, C)
    dy = torch.randn(1, l, h, p, generator=gen, dtype=F64)
    dse = torch.randn(1, h, l // C, p, n, generator=gen, dtype=F64)
    return dt, x, Bm, Cm, cum, dy, dse


def test_mamba2_intra_backward_is_the_vjp_of_m3():
    for C in (256, 128):
        dt, x, Bm, Cm, cum, dy, dse = _mamba2_case(C=C)
        got = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum, dy, dse, C)
        leaves = [t.clone().requires_grad_(True) for t in (dt, x, Bm, Cm, cum)]
        y, se = om.intra_chunk_ssd(*leaves, C)
        ref = torch.autograd.grad((y, se), leaves, (dy, dse))
        for name, a, c in zip(("ddt", "dx", "dB", "dC", "dcum"), got, ref):
            assert _rel(a, c) < 1e-11, (C, name)


def test_mamba2_intra_backward_mistake_is_caught(monkeypatch):
    """The clip mask of the decay to the chunk end applied as its complement
    (every in-range pair masked out) changes dcum."""
    dt, x, Bm, Cm, cum, dy, dse = _mamba2_case(seed=6)
    good = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum, dy, dse, 256)
    real = om.clip_mask
    monkeypatch.setattr(om, "clip_mask", lambda v, lo, hi: 1.0 - real(v, lo, hi))
    bad = om.intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum, dy, dse, 256)
    assert _rel(bad[4], good[4]) > 1e-3


def _mamba2_staged(dt, A, Bm, Cm, x, C, do, dsf, s0):
    """_mamba2_core_bwd (kernel_mamba2_trainable_B6.py:83-131) from the stages."""
    b, l, h, p = dt.shape
    ddt_p, dB, dC, dx, ds0, dcum = om.mamba2_bwd_scan(dt, A, Bm, Cm, x, C, do, dsf, s0)
    dtp = dt.reshape(b, l // C, C, h, p).permute(0, 3, 1, 2, 4)
    ddt2, dA = om.mamba2_dA_backward(dtp, A, dcum, C)
    ddt = ddt_p + ddt2.permute(0, 2, 3, 1, 4).reshape(b, l, h, p)
    return tuple(om.final_sanitize(t) for t in (ddt, dB, dC, dx, dA, ds0))


def _mamba2_full_case(seed=3, l=512, h=2, p=8, n=6):
    gen = torch.Generator().manual_seed(seed)
    dt = torch.nn.functional.softplus(torch.randn(1, l, h, p, generator=gen, dtype=F64) - 3)
    x = torch.randn(1, l, h, p, generator=gen, dtype=F64)
    Bm = torch.randn(1, l, n, generator=gen, dtype=F64) / n ** 0.5
    Cm = torch.randn(1, l, n, generator=gen, dtype=F64) / n ** 0.5
    A = -0.5 * torch.rand(h, generator=gen, dtype=F64)
    do = torch.randn(1, l, h, p, generator=gen, dtype=F64)
    dsf = 0.3 * torch.randn(1, h, p, n, generator=gen, dtype=F64)
    s0 = 0.3 * torch.randn(1, h, p, n, generator=gen, dtype=F64)
    return dt, A, Bm, Cm, x, do, dsf, s0


def test_mamba2_backward_stages_compose_to_mb0():
    """MB1 + MB2 + MB3 (mamba2_bwd_scan) and MB4 (mamba2_dA_backward), composed
    as the trainable op does, equal MB0's per-chunk backward (itself pinned
    against autograd and finite differences) at chunks 64, 128 and 256."""
    dt, A, Bm, Cm, x, do, dsf, s0 = _mamba2_full_case()
    for C in (64, 128, 256):
        got = _mamba2_staged(dt, A, Bm, Cm, x, C, do, dsf, s0)
        ref = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, do, dsf, s0)
        ref = tuple(om.final_sanitize(t) for t in ref)
        for name, a, c in zip(("ddt", "dB", "dC", "dx", "dA", "dstate0"), got, ref):
            assert _rel(a, c) < 1e-11, (C, name)


def test_mamba2_backward_stage_mistakes_are_caught(monkeypatch):
    dt, A, Bm, Cm, x, do, dsf, s0 = _mamba2_full_case(seed=9)
    ref = tuple(om.final_sanitize(t) for t in om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, 128, do, dsf, s0))

    def worst():
        got = _mamba2_staged(dt, A, Bm, Cm, x, 128, do, dsf, s0)
        return max(_rel(a, c) for a, c in zip(got, ref))

    # (1) MB1 without the carried state's decay term on the last row
    real = om.state_only_bwd

    def no_last_row(state_prev, C_c, cum, dy_off, carry, dtype=F64):
        dC, dp, dcum = real(state_prev, C_c, cum, dy_off, carry, dtype=dtype)
        d0 = real(state_prev, C_c, cum, dy_off, torch.zeros_like(carry), dtype=dtype)[2]
        dcum = dcum.clone()
        dcum[:, -1] = d0[:, -1]
        return dC, dp, dcum
    monkeypatch.setattr(om, "state_only_bwd", no_last_row)
    assert worst() > 1e-6
    monkeypatch.undo()

    # (2) MB4 with a forward instead of a reverse cumsum
    def forward_cumsum(dt_p, A_, dcum, C, dtype=F64):
        f = dtype
        raw = dt_p.to(f) * A_.to(f)[None, :, None, None, None]
        d = torch.cumsum(dcum.to(f), 3) * om.clip_mask(raw, -20.0, 20.0)
        return om.sanitize(d * A_.to(f)[None, :, None, None, None]), om.sanitize((d * dt_p.to(f)).sum((0, 2, 3, 4)))
    monkeypatch.setattr(om, "mamba2_dA_backward", forward_cumsum)
    assert worst() > 1e-6


def test_mamba2_state_only_backward_masks_on_the_clipped_exponent():
    """MB1's state-only step masks the y_off decay term on the clipped
    exponent clip(cum, -20, 0) (mamba2_bwd_state_reference.py:123-124), which
    every cum passes; MB0 masks on cum itself (mamba2_bwd_reference.py:131).
    With every cum >= 0 the decay is exp(0) = 1, so the step's dcum is
    exactly dy * (C state^T) on every row but the last (whose extra term is
    masked off on cum > 0), a closed form MB0's mask (all zeros there) fails."""
    gen = torch.Generator().manual_seed(23)
    b, Cs, h, p, n = 1, 16, 2, 8, 4
    sp = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    Cc = torch.randn(b, Cs, n, generator=gen, dtype=F64)
    cum = torch.rand(b, Cs, h, p, generator=gen, dtype=F64).cumsum(1)       # > 0
    dy = torch.randn(b, Cs, h, p, generator=gen, dtype=F64)
    carry = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    _, _, dcum = om.state_only_bwd(sp, Cc, cum, dy, carry)
    y_off = torch.einsum("bis,bhds->bihd", Cc, sp)
    assert torch.allclose(dcum, dy * y_off, rtol=0, atol=1e-12)
