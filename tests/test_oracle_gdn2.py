"""Pins the GDN2 oracle (oracle/gdn2.py) without running the reference.

Each check is chosen so that a plausible transcription mistake (a dropped
decay term, a wrong triangle, a transposed operand, a missing erase term)
fails at least one of them; ``test_planted_mistakes_are_caught`` plants such
mistakes in the oracle and asserts the checks catch them.
"""
import math

import pytest
import torch

from oracle import gdn2 as og

F64 = torch.float64


def _inputs(B, T, H, K, V, seed=0, g_scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen, dtype=F64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=F64)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(B, T, H, V, generator=gen, dtype=F64)
    b = torch.sigmoid(torch.randn(B, T, H, K, generator=gen, dtype=F64))
    w = torch.sigmoid(torch.randn(B, T, H, V, generator=gen, dtype=F64))
    g = torch.nn.functional.logsigmoid(3.0 + torch.randn(B, T, H, K, generator=gen, dtype=F64)) * g_scale
    return q, k, v, g, b, w


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def test_chunked_matches_token_serial():
    q, k, v, g, b, w = _inputs(2, 64, 2, 8, 6, seed=1)
    gen = torch.Generator().manual_seed(7)
    h0 = 0.3 * torch.randn(2, 2, 8, 6, generator=gen, dtype=F64)
    for scale in (1.0, 8 ** -0.5):
        o_c, h_c = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 16, h0=h0)
        o_s, h_s = og.gdn2_token_serial_reference(q, k, v, g, b, w, scale, h0=h0)
        assert _rel(o_c, o_s) < 1e-12
        assert _rel(h_c, h_s) < 1e-12


@pytest.mark.parametrize("chunks", [(4, 8, 16, 32)])
def test_chunk_size_invariance(chunks):
    q, k, v, g, b, w = _inputs(1, 64, 2, 8, 8, seed=2)
    ref = None
    for C in chunks:
        o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, C)
        if ref is None:
            ref = (o, h)
        else:
            assert _rel(o, ref[0]) < 1e-12
            assert _rel(h, ref[1]) < 1e-12


def test_state_passing_split_sequence():
    q, k, v, g, b, w = _inputs(1, 64, 3, 8, 4, seed=3)
    o_full, h_full = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 16)
    first = [t[:, :32] for t in (q, k, v, g, b, w)]
    second = [t[:, 32:] for t in (q, k, v, g, b, w)]
    o1, h1 = og.gdn2_chunked_wy_reference(*first, 1.0, 16)
    o2, h2 = og.gdn2_chunked_wy_reference(*second, 1.0, 16, h0=h1)
    assert _rel(torch.cat([o1, o2], 1), o_full) < 1e-13
    assert _rel(h2, h_full) < 1e-13


def test_wy_inverse_is_inverse():
    gen = torch.Generator().manual_seed(4)
    Akk = torch.tril(torch.randn(3, 32, 32, generator=gen, dtype=F64), diagonal=-1) * 0.2
    A = og.wy_inverse(Akk)
    eye = torch.eye(32, dtype=F64)
    assert (((eye + Akk) @ A) - eye).abs().max().item() < 1e-10
    assert torch.equal(torch.triu(A, 1), torch.zeros_like(A))


def test_closed_form_causal_linear_attention():
    """g=0, b=0, w=1: no decay, no erase -> o = tril(scale Q K^T) V."""
    q, k, v, g, b, w = _inputs(2, 32, 2, 8, 5, seed=5)
    g = torch.zeros_like(g)
    b = torch.zeros_like(b)
    w = torch.ones_like(w)
    scale = 0.7
    o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 8)
    qh, kh, vh = (t.permute(0, 2, 1, 3) for t in (q, k, v))
    att = torch.tril(scale * qh @ kh.transpose(-1, -2))
    o_ref = (att @ vh).permute(0, 2, 1, 3)
    assert _rel(o, o_ref) < 1e-12
    assert _rel(h, kh.transpose(-1, -2) @ vh) < 1e-12


def test_closed_form_single_token():
    """T=1, h0=0: o = scale (q.k) (w*v), h = k (w*v)^T."""
    q, k, v, g, b, w = _inputs(2, 1, 3, 6, 4, seed=6)
    scale = 1.3
    o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 1)
    qk = (q * k).sum(-1, keepdim=True)
    assert _rel(o, scale * qk * (w * v)) < 1e-13
    assert _rel(h, torch.einsum("bhk,bhv->bhkv", k[:, 0], (w * v)[:, 0])) < 1e-13


def test_decay_only_closed_form():
    """b=0, w=1, one channel: the state is a decayed sum, o_t = sum_s
    scale q_t k_s exp(gc_t - gc_s) v_s -- checks the decay exponent sign and
    the cumulative-sum reset at chunk boundaries."""
    q, k, v, g, b, w = _inputs(1, 24, 1, 1, 1, seed=8)
    q = torch.ones_like(q)
    k = torch.ones_like(k)
    b = torch.zeros_like(b)
    w = torch.ones_like(w)
    o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 8)
    G = torch.cumsum(g[0, :, 0, 0], 0)
    T = 24
    o_ref = torch.zeros(T, dtype=F64)
    for t in range(T):
        for s in range(t + 1):
            o_ref[t] += math.exp(G[t] - G[s]) * v[0, s, 0, 0]
    assert _rel(o[0, :, 0, 0], o_ref) < 1e-12


def _loss(q, k, v, w, b, g, h0, scale, C, dO, dH):
    o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, C, h0=h0)
    return (o * dO).sum() + (h * dH).sum()


def test_autodiff_matches_finite_differences():
    B, T, H, K, V, C = 1, 8, 1, 3, 2, 4
    q, k, v, g, b, w = _inputs(B, T, H, K, V, seed=9)
    gen = torch.Generator().manual_seed(10)
    h0 = 0.2 * torch.randn(B, H, K, V, generator=gen, dtype=F64)
    dO = torch.randn(B, T, H, V, generator=gen, dtype=F64)
    dH = torch.randn(B, H, K, V, generator=gen, dtype=F64)
    grads = og.gdn2_backward_autodiff(q, k, v, w, b, g, 0.9, C, dO, dH, h0=h0)
    prims = [q, k, v, w, b, g, h0]
    eps = 1e-6
    for i, x in enumerate(prims):
        d = torch.randn(x.shape, generator=gen, dtype=F64)
        plus = [p.clone() for p in prims]
        minus = [p.clone() for p in prims]
        plus[i] = x + eps * d
        minus[i] = x - eps * d
        fd = (_loss(*plus, 0.9, C, dO, dH) - _loss(*minus, 0.9, C, dO, dH)) / (2 * eps)
        an = (grads[i] * d).sum()
        assert abs(fd.item() - an.item()) < 1e-7 * max(1.0, abs(fd.item())), i


def test_hand_chain_matches_autodiff():
    B, T, H, K, V, C = 2, 32, 2, 8, 6, 8
    q, k, v, g, b, w = _inputs(B, T, H, K, V, seed=11)
    gen = torch.Generator().manual_seed(12)
    h0 = 0.2 * torch.randn(B, H, K, V, generator=gen, dtype=F64)
    dO = torch.randn(B, T, H, V, generator=gen, dtype=F64)
    dH = torch.randn(B, H, K, V, generator=gen, dtype=F64)
    for scale in (1.0, 0.35):
        ad = og.gdn2_backward_autodiff(q, k, v, w, b, g, scale, C, dO, dH, h0=h0)
        ch, _ = og.gdn2_backward_chain(q, k, v, w, b, g, scale, C, dO, dH, h0=h0)
        for name, a, c in zip("q k v w b g h0".split(), ad, ch):
            assert _rel(c, a) < 1e-10, name


def test_planted_mistakes_are_caught(monkeypatch):
    """Plant plausible mistakes in the oracle and check the pins catch them."""
    q, k, v, g, b, w = _inputs(1, 32, 1, 6, 4, seed=13)
    o_s, _ = og.gdn2_token_serial_reference(q, k, v, g, b, w, 1.0)

    # (1) first-order WY inverse (drops the T^2.. terms)
    monkeypatch.setattr(og, "wy_inverse", lambda Akk: torch.eye(Akk.shape[-1], dtype=Akk.dtype) - Akk)
    o_bad, _ = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 8)
    assert _rel(o_bad, o_s) > 1e-6
    monkeypatch.undo()

    # (2) decay sign flipped on the carried-state read (qg = q * exp(-gc))
    real = og.build_chunk_wy

    def flipped(*a, **kw):
        st = real(*a, **kw)
        st["qg"] = a[0].to(torch.float64) * torch.exp(-st["gc"])
        return st
    monkeypatch.setattr(og, "build_chunk_wy", flipped)
    o_bad, _ = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 8)
    assert _rel(o_bad, o_s) > 1e-6
    monkeypatch.undo()

    # (3) Akk with the diagonal included (causal instead of strict)
    def diag_kept(*a, **kw):
        st = real(*a, **kw)
        gc = st["gc"]
        kk = a[1].to(torch.float64)
        bk = a[4].to(torch.float64) * kk
        dd = torch.exp(gc[..., :, None, :] - gc[..., None, :, :])
        Akk = torch.einsum("...id,...ijd,...jd->...ij", bk, dd, kk) * torch.tril(torch.ones(8, 8, dtype=torch.float64))
        A = torch.linalg.inv(torch.eye(8, dtype=torch.float64) + Akk)
        st["w_pseudo"] = A @ st["kb_decayed"]
        st["u"] = A @ st["wv"]
        return st
    monkeypatch.setattr(og, "build_chunk_wy", diag_kept)
    o_bad, _ = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 8)
    assert _rel(o_bad, o_s) > 1e-6


def test_inter_chunk_combine_reproduces_the_chunked_reference():
    """Kernel D's restatement fed with the chunked reference's own per-chunk
    stages gives its o and h_final (the combine is the reference's scan step
    over those stages); a NaN / +-inf / beyond-1e4 h0 is sanitised first."""
    B, T, H, K, C = 1, 192, 2, 8, 64
    gen = torch.Generator().manual_seed(17)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)
    q, k = torch.nn.functional.normalize(r(B, T, H, K), dim=-1), torch.nn.functional.normalize(r(B, T, H, K), dim=-1)
    v, w = r(B, T, H, K), torch.sigmoid(r(B, T, H, K))
    b, g = torch.sigmoid(r(B, T, H, K)), torch.nn.functional.logsigmoid(r(B, T, H, K) + 3.0)
    h0 = 0.5 * r(B, H, K, K)
    o, h, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 0.7, C, h0=h0, return_stages=True)
    stack = lambda name: torch.stack([s[name] for s in st], 2)
    o_c, h_c = og.gdn2_inter_chunk_combine(stack("Aqk"), stack("w_pseudo"), stack("u"), stack("kg"), stack("qg"),
                                           stack("gc_last"), 0.7, h0=h0)
    o_c = o_c.permute(0, 2, 3, 1, 4).reshape(B, T, H, K)
    assert torch.allclose(o_c, o, rtol=0, atol=1e-12) and torch.allclose(h_c, h, rtol=0, atol=1e-12)
    bad = h0.clone()
    bad[0, 0, 0, 0], bad[0, 0, 1, 1], bad[0, 1, 2, 2], bad[0, 1, 3, 3] = float("nan"), float("inf"), 5e4, -float("inf")
    o_b, h_b = og.gdn2_inter_chunk_combine(stack("Aqk"), stack("w_pseudo"), stack("u"), stack("kg"), stack("qg"),
                                           stack("gc_last"), 0.7, h0=bad)
    clean = torch.nan_to_num(bad.clamp(-1e4, 1e4), nan=0.0, posinf=1e4, neginf=-1e4)
    o_r, h_r = og.gdn2_inter_chunk_combine(stack("Aqk"), stack("w_pseudo"), stack("u"), stack("kg"), stack("qg"),
                                           stack("gc_last"), 0.7, h0=clean)
    assert torch.equal(o_b, o_r) and torch.equal(h_b, h_r) and torch.isfinite(o_b).all()


# ------------------------------------------------------------------ the 256-row stage kernels
def _stage_blocks(t, BT):
    B, T, H, D = t.shape
    return t.reshape(B, T // BT, BT, H, D).permute(0, 3, 1, 2, 4)


def test_block_stages_compose_to_the_chunked_reference_at_256():
    """Kernels A (128-row sub-blocks), B (16-row block recursion, 128-row
    halves, A10 step), C and D at the reference's 256-row block, composed,
    equal the chunked reference at chunk 256; A's scores and C's arrays
    equal that reference's own per-chunk intermediates, and B's inverse its
    row-wise forward substitution."""
    q, k, v, g, b, w = _inputs(1, 512, 2, 16, 12, seed=21)
    scale = 0.7
    o_ref, h_ref, st = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, 256, return_stages=True)
    Aqk, Akk = og.chunk_scores(q, k, b, g, scale)
    assert Aqk.shape == (1, 2, 2, 256, 256)
    for n in range(2):
        assert _rel(Aqk[:, :, n], st[n]["Aqk"]) < 1e-12 and _rel(Akk[:, :, n], st[n]["Akk"]) < 1e-12
    A = og.wy_solve_blocked(Akk)
    assert _rel(A, og.wy_inverse(Akk)) < 1e-11
    eye = torch.eye(256, dtype=F64)
    assert ((eye + Akk) @ A - eye).abs().max().item() < 1e-10
    wp, u, kg, qg, gl = og.recompute_wy(q, k, v, w, b, g, A)
    for n in range(2):
        for name, x in (("w_pseudo", wp), ("u", u), ("kg", kg), ("qg", qg)):
            assert _rel(x[:, :, n], st[n][name]) < 1e-11, name
        assert _rel(gl[:, :, n], st[n]["gc_last"]) < 1e-12
    o, hf = og.gdn2_inter_chunk_combine(Aqk, wp, u, kg, qg, gl, scale)
    o = o.permute(0, 2, 3, 1, 4).reshape(o_ref.shape)
    assert _rel(o, o_ref) < 1e-11 and _rel(hf, h_ref) < 1e-11


def test_block_scores_sub_block_split_and_masks():
    """Kernel A's 128-row sub-blocks cover the block: the same scores at
    sub = 256 (one sub-block) and sub = 64; the strictly upper triangle of
    both and the diagonal of Akk are zero."""
    q, k, v, g, b, w = _inputs(1, 256, 1, 8, 8, seed=22)
    a128 = og.chunk_scores(q, k, b, g, 1.0)
    for sub in (256, 64):
        other = og.chunk_scores(q, k, b, g, 1.0, sub=sub)
        assert _rel(other[0], a128[0]) < 1e-13 and _rel(other[1], a128[1]) < 1e-13
    assert torch.count_nonzero(torch.triu(a128[0], 1)) == 0
    assert torch.count_nonzero(torch.triu(a128[1], 0)) == 0


def test_block_solve_sanitises_like_the_reference():
    """With a near-singular Akk the blocked solve's entries stay within
    +-1e4 and finite (every block product is sanitised), while the plain
    inverse of the same Akk overflows that range."""
    gen = torch.Generator().manual_seed(23)
    Akk = torch.tril(torch.randn(1, 256, 256, generator=gen, dtype=F64) * 3.0, -1)
    A = og.wy_solve_blocked(Akk)
    assert torch.isfinite(A).all() and A.abs().max().item() <= 1e4
    assert og.wy_inverse(Akk).abs().max().item() > 1e4
    # below the clip the two agree
    small = Akk * 0.01
    assert _rel(og.wy_solve_blocked(small), og.wy_inverse(small)) < 1e-12


def test_block_recompute_forms_w_v_in_float32():
    """Kernel C multiplies w and v after the upcast (kernel_c_recompute.py:53,
    64), the chunked reference before it (gdn2_wy_reference.py:94): with
    bf16 inputs the two u differ by the bf16 rounding of w v; with float64
    inputs they agree."""
    q, k, v, g, b, w = _inputs(1, 256, 1, 8, 8, seed=24)
    bf = [t.to(torch.bfloat16) for t in (q, k, v, b, w)]
    qb, kb, vb, bb, wb = bf
    _, _, st = og.gdn2_chunked_wy_reference(qb, kb, vb, g, bb, wb, 1.0, 256, return_stages=True)
    A = st[0]["A"][:, :, None]
    u_c = og.recompute_wy(qb, kb, vb, wb, bb, g, A)[1][:, :, 0]
    u_ref = st[0]["u"]
    wv32 = _stage_blocks(wb.double() * vb.double(), 256)[:, :, 0]
    assert _rel(u_c, og.sanitize(st[0]["A"] @ wv32)) < 1e-12
    assert 1e-5 < _rel(u_c, u_ref) < 2e-2
