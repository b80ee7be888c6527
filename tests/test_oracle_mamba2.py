"""Pins the Mamba2 SSD oracle (oracle/mamba2.py) without running the reference."""
import pytest
import torch

from oracle import mamba2 as om

F64 = torch.float64


def _inputs(b, l, h, p, n, seed=0, dt_mean=-2.0, a_max=16.0, dt_scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, l, h, p, generator=gen, dtype=F64)
    dt = torch.nn.functional.softplus(dt_mean + 0.5 * torch.randn(b, l, h, p, generator=gen, dtype=F64)) * dt_scale
    A = -torch.exp(torch.rand(h, generator=gen, dtype=F64) * torch.log(torch.tensor(a_max, dtype=F64)))
    Bm = torch.randn(b, l, n, generator=gen, dtype=F64) / n ** 0.5
    Cm = torch.randn(b, l, n, generator=gen, dtype=F64) / n ** 0.5
    return dt, A, Bm, Cm, x


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def test_chunked_matches_token_serial_clip_free():
    # per-step decay ~ -0.13 * |A|<=2 -> a 16-step chunk stays far inside +-20
    dt, A, Bm, Cm, x = _inputs(2, 64, 3, 5, 7, seed=1, a_max=2.0)
    gen = torch.Generator().manual_seed(2)
    s0 = 0.3 * torch.randn(2, 3, 5, 7, generator=gen, dtype=F64)
    y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, 16, state0=s0)
    y_t, s_t = om.mamba2_token_serial(dt, A, Bm, Cm, x, state0=s0)
    assert _rel(y, y_t) < 1e-12
    assert _rel(s, s_t) < 1e-12


def test_chunked_vs_token_serial_when_clip_fires_is_tiny():
    """At config-1 decay rates (A down to -16, 128-step chunks) the +-20
    pairwise clip fires; its floor exp(-20) changes the result only at the
    ~1e-9 level, which bounds what a kernel ignoring the floor can differ by."""
    dt, A, Bm, Cm, x = _inputs(1, 128, 4, 4, 8, seed=3, a_max=16.0)
    y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, 128)
    y_t, s_t = om.mamba2_token_serial(dt, A, Bm, Cm, x)
    err = _rel(y, y_t)
    assert 0 < err < 1e-6


def test_zero_decay_closed_form():
    """A = 0: y_i = sum_{j<=i} (C_i . B_j) dt_j x_j + C_i . s0 (a masked cumulative sum)."""
    dt, A, Bm, Cm, x = _inputs(2, 32, 2, 3, 4, seed=4)
    A = torch.zeros_like(A)
    gen = torch.Generator().manual_seed(5)
    s0 = torch.randn(2, 2, 3, 4, generator=gen, dtype=F64)
    y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, 8, state0=s0)
    CB = torch.tril(torch.einsum("bis,bjs->bij", Cm, Bm))
    y_ref = torch.einsum("bij,bjhp->bihp", CB, dt * x) + torch.einsum("bis,bhps->bihp", Cm, s0)
    assert _rel(y, y_ref) < 1e-12
    s_ref = s0 + torch.einsum("bjs,bjhp->bhps", Bm, dt * x)
    assert _rel(s, s_ref) < 1e-12


def test_chunk_size_invariance_clip_free():
    dt, A, Bm, Cm, x = _inputs(1, 64, 2, 4, 6, seed=6, a_max=1.5)
    ref = None
    for C in (8, 16, 32, 64):
        y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C)
        if ref is None:
            ref = (y, s)
        else:
            assert _rel(y, ref[0]) < 1e-12
            assert _rel(s, ref[1]) < 1e-12


def test_zero_state_split_identities():
    """state_prev = 0: y == y_diag and state_new == state_end
    (kernel_mamba2_b_intra.py:22-28)."""
    dt, A, Bm, Cm, x = _inputs(2, 16, 2, 3, 5, seed=7)
    zero = torch.zeros(2, 2, 3, 5, dtype=F64)
    y, s, parts = om.chunk_ssd(dt, A, Bm, Cm, x, zero)
    assert torch.equal(y, parts["y_diag"])
    assert torch.equal(s, parts["state_end"])


def _loss(dt, A, Bm, Cm, x, s0, C, dy, ds):
    y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0)
    return (y * dy).sum() + (s * ds).sum()


@pytest.mark.parametrize("a_max,C", [(2.0, 8), (16.0, 16)])
def test_mb0_matches_autodiff(a_max, C):
    """MB0 is designed to equal autodiff of the forward with straight-through
    clip masks (mamba2_bwd_reference.py:31-36); checked both clip-free and
    with the +-20 pairwise clip firing."""
    b, l, h, p, n = 2, 32, 2, 3, 4
    dt, A, Bm, Cm, x = _inputs(b, l, h, p, n, seed=8, a_max=a_max, dt_mean=-0.5)
    gen = torch.Generator().manual_seed(9)
    s0 = 0.5 * torch.randn(b, h, p, n, generator=gen, dtype=F64)
    dy = torch.randn(b, l, h, p, generator=gen, dtype=F64)
    ds = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    leaves = [t.clone().requires_grad_(True) for t in (dt, A, Bm, Cm, x, s0)]
    L = _loss(*leaves, C, dy, ds)
    ad = torch.autograd.grad(L, leaves)
    ddt, dB, dC, dx, dA, ds0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy, ds, state0=s0)
    for name, hand, auto in (("dt", ddt, ad[0]), ("A", dA, ad[1]), ("B", dB, ad[2]),
                             ("C", dC, ad[3]), ("x", dx, ad[4]), ("s0", ds0, ad[5])):
        assert _rel(hand, auto) < 1e-10, name


def test_mb0_matches_finite_differences():
    b, l, h, p, n, C = 1, 8, 2, 2, 3, 4
    dt, A, Bm, Cm, x = _inputs(b, l, h, p, n, seed=10, a_max=4.0, dt_mean=-0.5)
    gen = torch.Generator().manual_seed(11)
    s0 = 0.5 * torch.randn(b, h, p, n, generator=gen, dtype=F64)
    dy = torch.randn(b, l, h, p, generator=gen, dtype=F64)
    ds = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    ddt, dB, dC, dx, dA, ds0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy, ds, state0=s0)
    prims = [dt, A, Bm, Cm, x, s0]
    grads = [ddt, dA, dB, dC, dx, ds0]
    eps = 1e-6
    for i, xx in enumerate(prims):
        d = torch.randn(xx.shape, generator=gen, dtype=F64)
        plus = [p_.clone() for p_ in prims]
        minus = [p_.clone() for p_ in prims]
        plus[i] = xx + eps * d
        minus[i] = xx - eps * d
        fd = (_loss(*plus, C, dy, ds) - _loss(*minus, C, dy, ds)) / (2 * eps)
        an = (grads[i] * d).sum()
        assert abs(fd.item() - an.item()) < 1e-7 * max(1.0, abs(fd.item())), i


def test_planted_mistakes_are_caught(monkeypatch):
    b, l, h, p, n, C = 1, 16, 2, 2, 3, 8
    dt, A, Bm, Cm, x = _inputs(b, l, h, p, n, seed=12, a_max=2.0)
    y_t, _ = om.mamba2_token_serial(dt, A, Bm, Cm, x)

    # (1) forward: decay_to_end with its sign flipped
    real = om.chunk_ssd

    def chunk_bad(dt_c, A_, B_c, C_c, x_c, state_prev, dtype=F64):
        y_c, _, parts = real(dt_c, A_, B_c, C_c, x_c, state_prev, dtype)
        cum = parts["cumdecay"]
        dBx = dt_c.to(dtype) * x_c.to(dtype)
        wrong_end = torch.einsum("bcs,bchd->bhds", B_c.to(dtype), dBx * torch.exp(cum - cum[:, -1:]))
        dce = torch.exp(torch.clamp(cum[:, -1], -20.0, 0.0))
        return y_c, state_prev * dce[..., None] + wrong_end, parts
    monkeypatch.setattr(om, "chunk_ssd", chunk_bad)
    y_bad, _ = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C)
    assert _rel(y_bad, y_t) > 1e-6
    monkeypatch.undo()

    # (2) backward: the [-20, 0] window mask wrongly closed, which drops the
    # y_off decay term and the last-row decay_chunk_end term (:120, :131)
    gen = torch.Generator().manual_seed(3)
    dy = torch.randn(b, l, h, p, generator=gen, dtype=F64)
    ds = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    s0 = torch.randn(b, h, p, n, generator=gen, dtype=F64)
    leaves = [t.clone().requires_grad_(True) for t in (dt, A, Bm, Cm, x, s0)]
    ad = torch.autograd.grad(_loss(*leaves, C, dy, ds), leaves)
    good = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy, ds, state0=s0)
    assert _rel(good[0], ad[0]) < 1e-10 and _rel(good[4], ad[1]) < 1e-10
    real_mask = om.clip_mask
    monkeypatch.setattr(om, "clip_mask", lambda x_, lo, hi: torch.zeros_like(x_)
                        if (lo, hi) == (-20.0, 0.0) else real_mask(x_, lo, hi))
    bad = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy, ds, state0=s0)
    assert _rel(bad[0], ad[0]) > 1e-6
    assert _rel(bad[4], ad[1]) > 1e-6


# ---------------------------------------------------------------- stages M2 -> M3 -> M4
@pytest.mark.parametrize("C", [16, 32, 256])
def test_stages_compose_to_the_chunked_reference(C):
    """With every step exponent negative and a moderate state0 the stage
    kernels' clips never bind, so M2 -> M3 -> M4 equals the chunked reference
    (chunk 256: two 128-row sub-blocks inside M3)."""
    l = 512 if C == 256 else 64
    dt, A, Bm, Cm, x = _inputs(2, l, 3, 5, 7, seed=41)
    s0 = 0.3 * torch.randn(2, 3, 5, 7, generator=torch.Generator().manual_seed(42), dtype=F64)
    cum = om.build_chunk_cumdecay(dt, A, C)
    y_diag, state_end = om.intra_chunk_ssd(dt, x, Bm, Cm, cum, C)
    y, sf = om.mamba2_inter_chunk_combine(y_diag, state_end, cum, Cm, C, state0=s0)
    y_r, s_r, parts = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0, return_parts=True)
    assert _rel(y, y_r) < 1e-12 and _rel(sf, s_r) < 1e-12
    # the per-chunk stage arrays are the reference's own intermediates
    assert _rel(cum[:, :, 1], parts[1]["cumdecay"].permute(0, 2, 1, 3)) < 1e-12
    assert _rel(state_end[:, :, 1], parts[1]["state_end"]) < 1e-12


def test_single_chunk_y_diag_is_the_whole_output():
    """One chunk from a zero state: y_diag is y and state_end is the final
    state (the identity the reference's M3 docstring cross-checks)."""
    dt, A, Bm, Cm, x = _inputs(1, 32, 2, 4, 6, seed=43, a_max=2.0)   # no -20 clip fires
    cum = om.build_chunk_cumdecay(dt, A, 32)
    y_diag, state_end = om.intra_chunk_ssd(dt, x, Bm, Cm, cum, 32)
    y, s = om.mamba2_token_serial(dt, A, Bm, Cm, x)
    assert _rel(y_diag, y) < 1e-12 and _rel(state_end[:, :, 0], s) < 1e-12


@pytest.mark.parametrize("C", [8, 16])
def test_stage_m3_matches_element_loops_with_positive_exponents(C):
    """A positive step exponent (A > 0 for one head) drives the pair weights
    to exp(20) and the chunk's write past 1e4, where the stage kernel's clips
    (no 1e6 cap, a sanitised write) decide the result: the vectorised M3
    against the element-by-element restatement, and unlike the whole-path
    oracle's capped y_diag."""
    dt, A, Bm, Cm, x = _inputs(1, 2 * C, 2, 3, 4, seed=44)
    A[0] = 6.0
    dt = dt * 8.0
    cum = om.build_chunk_cumdecay(dt, A, C)
    y_diag, state_end = om.intra_chunk_ssd(dt, x, Bm, Cm, cum, C)
    y_l, se_l = om.intra_chunk_ssd_loops(dt, x, Bm, Cm, cum, C)
    assert _rel(y_diag, y_l) < 1e-12 and _rel(state_end, se_l) < 1e-12
    _, _, parts = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, return_parts=True)
    whole = torch.cat([q["y_diag"] for q in parts], 1)
    assert (y_diag - whole).abs().max().item() > 1.0


def test_stage_m4_sanitises_state0():
    """M4 clips state0 to +-1e4 and zeroes its NaNs (kernel_mamba2_c_interchunk.py:58)."""
    dt, A, Bm, Cm, x = _inputs(1, 32, 1, 2, 3, seed=45)
    cum = om.build_chunk_cumdecay(dt, A, 16)
    y_diag, state_end = om.intra_chunk_ssd(dt, x, Bm, Cm, cum, 16)
    s0 = torch.zeros(1, 1, 2, 3, dtype=F64)
    s0[0, 0, 0, 0], s0[0, 0, 1, 2] = float("nan"), 5e4
    y, sf = om.mamba2_inter_chunk_combine(y_diag, state_end, cum, Cm, 16, state0=s0)
    clean = s0.clone()
    clean[0, 0, 0, 0], clean[0, 0, 1, 2] = 0.0, 1e4
    y2, sf2 = om.mamba2_inter_chunk_combine(y_diag, state_end, cum, Cm, 16, state0=clean)
    assert torch.equal(y, y2) and torch.equal(sf, sf2) and torch.isfinite(y).all()
