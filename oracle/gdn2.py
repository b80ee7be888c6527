"""GDN2 (Gated DeltaNet-2) oracle: CPU restatement of the reference's WY forms.

Test infrastructure only (see ``oracle/__init__.py``).

Conventions (reference ``atomic_ops/gdn2_wy_reference.py``):
  q, k, b, g : [B, T, H, K]      (b = per-channel erase gate "beta")
  v, w       : [B, T, H, V]      (w = per-channel write gate)
  h          : [B, H, K, V]      fp32 state
  o          : [B, T, H, V]      returned in the compute dtype (fp32 in the
                                  reference, ``gdn2_wy_reference.py:151``)

All arithmetic runs in ``dtype`` (float64 by default).  Inputs that arrive in
bfloat16 are upcast on entry exactly like the reference's ``.astype(f32)``
(``gdn2_wy_reference.py:75-77``); the one product the reference forms in the
input dtype before upcasting, ``w_c * v_c`` (``:94``), is formed the same way.
"""
from __future__ import annotations

import torch

CLIP_DECAY = 20.0
CLIP_ACC = 1e4


def n2n(x):
    """``jnp.nan_to_num(x, nan=0, posinf=1e4, neginf=-1e4)`` (gdn2_wy_reference.py:86)."""
    return torch.nan_to_num(x, nan=0.0, posinf=CLIP_ACC, neginf=-CLIP_ACC)


def sanitize(x, c=CLIP_ACC):
    """clip to [-c, c] then nan_to_num (gdn2_wy_reference.py:141)."""
    return torch.nan_to_num(torch.clamp(x, -c, c), nan=0.0, posinf=c, neginf=-c)


def wy_inverse(Akk):
    """Row-wise forward substitution ``A[i] = e_i - Akk[i,:] @ A`` for a
    strictly lower triangular ``Akk`` (gdn2_wy_reference.py:16-30).

    Rows are built one at a time and stacked (no in-place writes) so torch
    autograd can differentiate through it, as ``jax.vjp`` does through the
    reference's ``lax.scan``."""
    C = Akk.shape[-1]
    eye = torch.eye(C, dtype=Akk.dtype, device=Akk.device)
    rows = []
    for i in range(C):
        if i == 0:
            rows.append(eye[0].expand(Akk.shape[:-2] + (C,)))
            continue
        prev = torch.stack(rows, dim=-2)                      # [..., i, C]
        contrib = torch.einsum("...j,...jk->...k", Akk[..., i, :i], prev)
        rows.append(eye[i] - contrib)
    return torch.stack(rows, dim=-2)


def build_chunk_wy(q_c, k_c, v_c, g_c, b_c, w_c, scale, dtype=torch.float64):
    """Per-chunk WY build (gdn2_wy_reference.py:59-102).

    Inputs are one chunk in [B, H, C, D] layout.  Returns a dict with
    ``gc, Aqk, Akk, A, w_pseudo, u, kg, qg, gc_last`` (all ``dtype``)."""
    f = dtype
    C = q_c.shape[-2]
    gc = torch.cumsum(g_c.to(f), dim=-2)                                  # :63
    decay_diff = gc[..., :, None, :] - gc[..., None, :, :]               # :66
    edecay = torch.exp(torch.clamp(decay_diff, -CLIP_DECAY, CLIP_DECAY))  # :70
    causal = torch.tril(torch.ones(C, C, dtype=f))                        # :72
    strict = torch.tril(torch.ones(C, C, dtype=f), diagonal=-1)          # :73
    q = q_c.to(f)
    k = k_c.to(f)
    b = b_c.to(f)
    Aqk = scale * torch.einsum("...id,...ijd,...jd->...ij", q, edecay, k) * causal   # :79
    bk = b * k                                                            # :80
    Akk = torch.einsum("...id,...ijd,...jd->...ij", bk, edecay, k) * strict         # :81
    Aqk = n2n(Aqk)                                                        # :86
    Akk = n2n(Akk)                                                        # :87
    A = n2n(wy_inverse(Akk))                                              # :89-90
    kb_decayed = bk * torch.exp(gc)                                       # :92
    wv = (w_c * v_c).to(f)                                                # :94 (product in input dtype)
    w_pseudo = n2n(A @ kb_decayed)                                        # :93,95
    u = n2n(A @ wv)                                                       # :94,96
    gc_last = gc[..., -1, :]                                              # :98
    kg = k * torch.exp(gc_last[..., None, :] - gc)                        # :99
    qg = q * torch.exp(gc)                                                # :100
    return dict(gc=gc, Aqk=Aqk, Akk=Akk, A=A, w_pseudo=w_pseudo, u=u, kg=kg,
                qg=qg, gc_last=gc_last, wv=wv, kb_decayed=kb_decayed)


def _to_chunks(t, C):
    """[B, T, H, D] -> [NT, B, H, C, D]."""
    B, T, H, D = t.shape
    return t.reshape(B, T // C, C, H, D).permute(1, 0, 3, 2, 4)


def _from_chunks(t):
    """[NT, B, H, C, D] -> [B, T, H, D]."""
    NT, B, H, C, D = t.shape
    return t.permute(1, 0, 3, 2, 4).reshape(B, NT * C, H, D)


def gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, chunk_size, h0=None,
                              dtype=torch.float64, return_stages=False):
    """Chunked WY forward (gdn2_wy_reference.py:105-152).

    Argument order follows the reference function (``q,k,v,g,b,w``), not the
    drop-in wrapper (``q,k,v,w,b,g``, kernel_trainable_B6.py:187)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    assert T % C == 0, f"seq_len={T} must be divisible by chunk_size={C}"   # :109
    f = dtype
    ch = [_to_chunks(t, C) for t in (q, k, v, g, b, w)]                    # :120
    h = torch.zeros(B, H, K, V, dtype=f) if h0 is None else h0.to(f)        # :122-123
    outs, stages = [], []
    for n in range(T // C):
        st = build_chunk_wy(*(t[n] for t in ch), scale, dtype=f)            # :127
        h_pre = h
        wh = st["w_pseudo"] @ h_pre                                         # :129
        v_new = st["u"] - wh                                                # :130
        qh = st["qg"] @ h_pre                                               # :132
        intra = st["Aqk"] @ v_new                                           # :134
        o_c = scale * qh + intra                                            # :136
        decay_h = torch.exp(st["gc_last"])[..., None]                       # :138
        write = st["kg"].transpose(-1, -2) @ v_new                          # :139
        h = sanitize(h_pre * decay_h + write)                               # :140-141
        o_c = n2n(o_c)                                                      # :142
        outs.append(o_c)
        if return_stages:
            st = dict(st, h_pre=h_pre, v_new=v_new, o=o_c)
            stages.append(st)
    o = _from_chunks(torch.stack(outs, 0))                                  # :151
    if return_stages:
        return o, h, stages
    return o, h


def gdn2_inter_chunk_combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None, dtype=torch.float64,
                             return_state=False):
    """Kernel D of the staged forward, ``gdn2_inter_chunk_combine``
    (kernel_d_pipeline.py:94-124), over per-chunk arrays in its layout:
    Aqk [B, H, NT, C, C]; w_pseudo, kg, qg [B, H, NT, C, K]; u [B, H, NT, C, V];
    gc_last [B, H, NT, K].  Returns o [B, H, NT, C, V] and h_final.  Unlike the
    chunked reference it sanitises h0 first (``_sanitize_h0``, :54-55,101).
    With ``return_state`` it also returns the state entering each chunk and
    v_new, [B, H, NT, K, V] and [B, H, NT, C, V]
    (``gdn2_inter_chunk_combine_with_state``, :127-158)."""
    f = dtype
    Aqk, w_pseudo, u, kg, qg, gc_last = (t.to(f) for t in (Aqk, w_pseudo, u, kg, qg, gc_last))
    B, H, NT, C, K = w_pseudo.shape
    V = u.shape[-1]
    h = torch.zeros(B, H, K, V, dtype=f) if h0 is None else sanitize(h0.to(f))   # :98-101
    outs, pres, vnews = [], [], []
    for n in range(NT):                                                        # :105-123
        h_pre = h
        v_new = u[:, :, n] - w_pseudo[:, :, n] @ h_pre
        o_c = scale * (qg[:, :, n] @ h_pre) + Aqk[:, :, n] @ v_new
        h = sanitize(h_pre * torch.exp(gc_last[:, :, n])[..., None] + kg[:, :, n].transpose(-1, -2) @ v_new)
        outs.append(n2n(o_c))
        if return_state:
            pres.append(h_pre)
            vnews.append(v_new)
    if return_state:
        return torch.stack(outs, 2), h, torch.stack(pres, 2), torch.stack(vnews, 2)
    return torch.stack(outs, 2), h


def _blocks(t, BT):
    """[B, T, H, D] -> [B, H, NT, BT, D] (reshape_in, kernel_a_scores.py:75-77)."""
    B, T, H, D = t.shape
    return t.reshape(B, T // BT, BT, H, D).permute(0, 3, 1, 2, 4)


def chunk_scores(q, k, b, g, scale, block=256, sub=128, dtype=torch.float64):
    """Kernel A, ``build_chunk_scores_pallas`` (kernel_a_scores.py:26-98):
    per block of ``block`` rows, gc = tril @ g (:32-34), and for each pair of
    ``sub``-row sub-blocks (si >= sj) the pairwise-decay scores with the
    causal / strict masks on diagonal sub-blocks and nan_to_num (:39-66).
    Returns (Aqk, Akk) [B, H, NT, block, block] in ``dtype``."""
    f = dtype
    q_, k_, b_, g_ = (_blocks(t.to(f), block) for t in (q, k, b, g))
    gc = torch.cumsum(g_, dim=-2)                                              # :32-34
    Aqk = torch.zeros(q_.shape[:-1] + (block,), dtype=f)
    Akk = torch.zeros_like(Aqk)
    idx = torch.arange(sub)
    causal = (idx[:, None] >= idx[None, :]).to(f)
    strict = (idx[:, None] > idx[None, :]).to(f)
    for si in range(block // sub):                                             # :39-40
        for sj in range(si + 1):
            i0, j0 = si * sub, sj * sub
            dd = gc[..., i0:i0 + sub, None, :] - gc[..., None, j0:j0 + sub, :]  # :51
            e = torch.exp(torch.clamp(dd, -CLIP_DECAY, CLIP_DECAY))             # :52
            qi, ki, bi, kj = (t[..., r0:r0 + sub, :] for t, r0 in ((q_, i0), (k_, i0), (b_, i0), (k_, j0)))
            aqk = scale * torch.einsum("...id,...ijd,...jd->...ij", qi, e, kj)  # :54
            akk = torch.einsum("...id,...ijd,...jd->...ij", bi * ki, e, kj)     # :55-56
            if si == sj:                                                      # :58-63
                aqk = aqk * causal
                akk = akk * strict
            Aqk[..., i0:i0 + sub, j0:j0 + sub] = n2n(aqk)                     # :65
            Akk[..., i0:i0 + sub, j0:j0 + sub] = n2n(akk)                     # :66
    return Aqk, Akk


def _micro_forward_substitution(T):
    """One MB x MB block (kernel_b_solve.py:66-87): row i of A is
    sanitize(e_i - T[i, :] @ A) with the rows >= i of A still zero."""
    MB = T.shape[-1]
    eye = torch.eye(MB, dtype=T.dtype)
    A = torch.zeros_like(T)
    for i in range(MB):
        contrib = torch.einsum("...j,...jc->...c", T[..., i, :], A)           # :78-79
        A = A.clone()
        A[..., i, :] = sanitize(eye[i] - contrib)                             # :80-83
    return A


def _block_solve(T, mb=16):
    """(I + T)^-1 of one strictly lower [.., BC, BC] block by the MB = 16
    block recursion (kernel_b_solve.py:90-127), sanitising every block
    product and accumulation."""
    BC = T.shape[-1]
    nm = BC // mb
    sl = lambda i: slice(i * mb, (i + 1) * mb)
    blocks = {}
    for m in range(nm):
        A_mm = sanitize(_micro_forward_substitution(T[..., sl(m), sl(m)]))    # :104
        blocks[m, m] = A_mm
        for n in range(m - 1, -1, -1):                                        # :107
            acc = torch.zeros_like(A_mm)
            for kk in range(n, m):                                            # :108-113
                acc = sanitize(acc + T[..., sl(m), sl(kk)] @ blocks[kk, n])
            blocks[m, n] = sanitize(-(A_mm @ acc))                            # :114-116
    A = torch.zeros_like(T)
    for (m, n), blk in blocks.items():                                        # :118-127
        A[..., sl(m), sl(n)] = blk
    return A


def wy_solve_blocked(Akk, sub=128):
    """Kernel B, ``wy_solve_pallas`` (kernel_b_solve.py:130-171): the two
    ``sub``-row halves by ``_block_solve``, then A10 = sanitize(-A11
    sanitize(T10 A00)).  Akk [..., 2 sub, 2 sub]; the upper-right block of
    the result is zero."""
    T00 = Akk[..., :sub, :sub]
    T11 = Akk[..., sub:, sub:]
    T10 = Akk[..., sub:, :sub]
    A00 = _block_solve(T00)                                                   # :137
    A11 = _block_solve(T11)                                                   # :138
    tmp = sanitize(T10 @ A00)                                                 # :140-141
    A10 = sanitize(-(A11 @ tmp))                                              # :142-143
    A = torch.zeros_like(Akk)
    A[..., :sub, :sub] = A00                                                  # :145-148
    A[..., sub:, :sub] = A10
    A[..., sub:, sub:] = A11
    return A


def recompute_wy(q, k, v, w, b, g, A, dtype=torch.float64):
    """Kernel C, ``recompute_wy_pallas`` (kernel_c_recompute.py:48-82) at the
    block of A ([B, H, NT, BT, BT]): w_pseudo = A (b k e^gc), u = A (w v)
    with w v formed after the upcast (:49-56,64), kg = k e^(gc_last - gc),
    qg = q e^gc, gc_last, each sanitised to +-1e4.  Returns
    (w_pseudo, u, kg, qg, gc_last)."""
    f = dtype
    BT = A.shape[-1]
    q_, k_, v_, w_, b_, g_ = (_blocks(t.to(f), BT) for t in (q, k, v, w, b, g))
    gc = torch.cumsum(g_, dim=-2)                                              # :58-60
    kb_decayed = b_ * k_ * torch.exp(gc)                                       # :62
    A = A.to(f)
    w_pseudo = sanitize(A @ kb_decayed)                                        # :63,68
    u = sanitize(A @ (w_ * v_))                                                # :64,69
    gl = gc[..., -1, :]                                                        # :71
    kg = sanitize(k_ * torch.exp(gl[..., None, :] - gc))                       # :72,80
    qg = sanitize(q_ * torch.exp(gc))                                          # :73,81
    return w_pseudo, u, kg, qg, sanitize(gl)                                   # :82


def gdn2_token_serial_reference(q, k, v, g, b, w, scale, h0=None, dtype=torch.float64):
    """Token-serial recurrence (gdn2_wy_reference.py:33-56), an independent
    oracle for the chunked form.  Returns o in ``dtype`` (the reference casts
    to the input dtype at :55; the tests compare in float64)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    f = dtype
    alpha = torch.exp(g.to(f))                                               # :38
    h = torch.zeros(B, H, K, V, dtype=f) if h0 is None else h0.to(f)
    outs = []
    for t in range(T):
        h = h * alpha[:, t, :, :, None]                                      # :45
        bk = (b[:, t] * k[:, t]).to(f)                                       # :46
        erase = torch.einsum("bhd,bhdv->bhv", bk, h)                          # :47
        v_new = (w[:, t] * v[:, t]).to(f) - erase                             # :48
        h = h + torch.einsum("bhd,bhv->bhdv", k[:, t].to(f), v_new)           # :49
        outs.append(torch.einsum("bhdv,bhd->bhv", h, (q[:, t] * scale).to(f)))  # :50
    return torch.stack(outs, 1), h


def final_sanitize(x):
    """``_final_sanitize`` at the custom_vjp boundary (kernel_trainable_B6.py:64-66)."""
    return sanitize(x, CLIP_ACC)


def gdn2_backward_autodiff(q, k, v, w, b, g, scale, chunk_size, do, dh_final=None,
                           h0=None, dtype=torch.float64):
    """The GDN2 gradient as the reference defines it: ``jax.vjp`` of the
    chunked WY reference followed by ``_final_sanitize``
    (kernel_trainable.py:38-55; argument remap at :42-43).  Takes the
    drop-in argument order ``q,k,v,w,b,g``.  Returns
    ``(dq, dk, dv, dw, db, dg, dh0)`` in ``dtype``."""
    f = dtype
    B, T, H, K = q.shape
    V = v.shape[-1]
    leaves = [t.detach().to(f).requires_grad_(True) for t in (q, k, v, w, b, g)]
    h0_ = torch.zeros(B, H, K, V, dtype=f) if h0 is None else h0.detach().to(f)
    h0_.requires_grad_(True)
    # The reference upcasts every input on entry; w*v is the one product it
    # forms before the upcast.  For float64 leaves the two coincide.
    qf, kf, vf, wf, bf, gf = leaves
    o, h_fin = gdn2_chunked_wy_reference(qf, kf, vf, gf, bf, wf, scale, chunk_size,
                                         h0=h0_, dtype=f)
    dO = do.to(f)
    dH = torch.zeros_like(h_fin) if dh_final is None else dh_final.to(f)
    grads = torch.autograd.grad((o, h_fin), leaves + [h0_], (dO, dH), allow_unused=True)
    grads = [torch.zeros_like(x) if gr is None else gr for gr, x in zip(grads, leaves + [h0_])]
    return tuple(final_sanitize(gr) for gr in grads)


def gdn2_backward_chain(q, k, v, w, b, g, scale, chunk_size, do, dh_final=None,
                        h0=None, dtype=torch.float64):
    """Hand restatement of the B2 -> B1 -> B3 -> B4 -> B5 chain
    (kernel_trainable_B6.py:97-181) at chunk ``chunk_size``.

    Independent of autograd: used to pin ``gdn2_backward_autodiff`` and to
    give per-stage intermediates for kernel-level tests.  Returns the final
    gradients ``(dq, dk, dv, dw, db, dg, dh0)`` and a dict of per-chunk
    intermediates."""
    f = dtype
    C = chunk_size
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    o, h_fin, st = gdn2_chunked_wy_reference(q, k, v, g, b, w, scale, C, h0=h0,
                                             dtype=f, return_stages=True)
    do_ch = _to_chunks(do.to(f), C)
    qc, kc, vc, gc_in, bc, wc = (_to_chunks(t, C) for t in (q, k, v, g, b, w))
    causal = torch.tril(torch.ones(C, C, dtype=f))
    strict = torch.tril(torch.ones(C, C, dtype=f), diagonal=-1)

    # B2 (kernel_bwd_b2_dav.py:61-73)
    dAqk = [n2n((do_ch[n] @ st[n]["v_new"].transpose(-1, -2)) * causal) for n in range(NT)]
    dv_partial = [n2n(st[n]["Aqk"].transpose(-1, -2) @ do_ch[n]) for n in range(NT)]

    # B1 reverse scan (kernel_bwd_b1_dhu.py:14-44)
    dh = torch.zeros(B, H, K, V, dtype=f) if dh_final is None else dh_final.to(f)
    dh = sanitize(dh)                                                        # b1:18
    dh_next = [None] * NT
    dv_all = [None] * NT
    for n in reversed(range(NT)):
        s = st[n]
        dh_next[n] = dh
        decay = torch.exp(s["gc_last"])[..., None]                            # b1:24
        from_out = s["qg"].transpose(-1, -2) @ (scale * do_ch[n])             # b1:26-27
        dv_new = sanitize(dv_partial[n] + s["kg"] @ dh)                       # b1:30-32
        from_vnew = -(s["w_pseudo"].transpose(-1, -2) @ dv_new)               # b1:34
        dh = sanitize(from_out + dh * decay + from_vnew)                      # b1:36-37
        dv_all[n] = dv_new
    dh0 = dh

    outs = {k_: [] for k_ in ("dq", "dk", "db", "dw", "dv", "dg")}
    dAkk_all = []
    for n in range(NT):
        s = st[n]
        qf, kf, bf_, wf, vf = (t[n].to(f) for t in (qc, kc, bc, wc, vc))
        gc = s["gc"]
        gcl = s["gc_last"]
        A = s["A"]
        h_pre = s["h_pre"]
        v_new = s["v_new"]
        dO = do_ch[n]
        dv = dv_all[n]
        dhn = dh_next[n]
        # B3 (kernel_bwd_b3_wy_dqkg.py:128-213)
        egc = torch.exp(gc)
        kb_dec = bf_ * kf * egc
        kg = kf * torch.exp(gcl[..., None, :] - gc)
        qg = qf * egc
        wv = s["wv"]
        dqg = (scale * dO) @ h_pre.transpose(-1, -2)
        dw_pseudo = (-dv) @ h_pre.transpose(-1, -2)
        dkg = v_new @ dhn.transpose(-1, -2)
        dA_total = dw_pseudo @ kb_dec.transpose(-1, -2) + dv @ wv.transpose(-1, -2)
        dkb = A.transpose(-1, -2) @ dw_pseudo
        dwv = A.transpose(-1, -2) @ dv
        dA_total = sanitize(dA_total)
        tmp = sanitize(dA_total @ A.transpose(-1, -2))
        dAkk = n2n(-(A.transpose(-1, -2) @ tmp) * strict)
        dAkk_all.append(dAkk)
        dk3 = dkb * egc * bf_ + dkg * torch.exp(gcl[..., None, :] - gc)
        db3 = dkb * egc * kf
        dx = dkg * kg
        dgc3 = dkb * kb_dec + dqg * qg - dx
        dgc_last = dx.sum(-2) + torch.exp(gcl) * (dhn * h_pre).sum(-1)
        dgc3 = dgc3.clone()
        dgc3[..., -1, :] = dgc3[..., -1, :] + dgc_last
        dq3 = dqg * egc
        dw3 = dwv * vf
        dv3 = dwv * wf
        dq3, dk3, db3, dw3, dv3, dgc3 = map(n2n, (dq3, dk3, db3, dw3, dv3, dgc3))
        # B4 (kernel_bwd_b4_intra.py:57-132), full chunk as one block
        diff = gc[..., :, None, :] - gc[..., None, :, :]
        clipmask = ((diff >= -CLIP_DECAY) & (diff <= CLIP_DECAY)).to(f)
        E = torch.exp(torch.clamp(diff, -CLIP_DECAY, CLIP_DECAY))
        dMqk = dAqk[n] * causal
        dMkk = dAkk * strict
        Lqk = scale * qf
        bk = bf_ * kf
        dL_qk = torch.einsum("...ij,...ijd,...jd->...id", dMqk, E, kf)
        dR_qk = torch.einsum("...ij,...ijd,...id->...jd", dMqk, E, Lqk)
        wq = dMqk[..., None] * Lqk[..., :, None, :] * kf[..., None, :, :] * E * clipmask
        dL_kk = torch.einsum("...ij,...ijd,...jd->...id", dMkk, E, kf)
        dR_kk = torch.einsum("...ij,...ijd,...id->...jd", dMkk, E, bk)
        wk = dMkk[..., None] * bk[..., :, None, :] * kf[..., None, :, :] * E * clipmask
        dgc4 = wq.sum(-2) - wq.sum(-3) + wk.sum(-2) - wk.sum(-3)
        dq4 = sanitize(dL_qk * scale)
        dk4 = sanitize(dR_qk + dR_kk + dL_kk * bf_)
        db4 = sanitize(dL_kk * kf)
        dgc4 = sanitize(dgc4)
        # combine + B5 reverse cumsum (kernel_bwd_b5_reverse_cumsum.py:17-24)
        dgc_total = dgc3 + dgc4
        dg = sanitize(torch.flip(torch.cumsum(torch.flip(dgc_total, [-2]), -2), [-2]))
        outs["dq"].append(dq3 + dq4)
        outs["dk"].append(dk3 + dk4)
        outs["db"].append(db3 + db4)
        outs["dw"].append(dw3)
        outs["dv"].append(dv3)
        outs["dg"].append(dg)
    res = {k_: final_sanitize(_from_chunks(torch.stack(vv, 0))) for k_, vv in outs.items()}
    inter = dict(dAqk=dAqk, dAkk=dAkk_all, dv_partial=dv_partial, dh_next=dh_next, dv_new=dv_all,
                 stages=st)
    return (res["dq"], res["dk"], res["dv"], res["dw"], res["db"], res["dg"],
            final_sanitize(dh0)), inter


# ---------------------------------------------------------------- backward stages
# The staged backward of the reference's trainable op (kernel_trainable_B6.py:
# 97-181) at its Pallas block: kernels B2, B1, B3, B4, B5 over per-block
# arrays [B, H, NT, BT, *].  Each follows its reference kernel's clip /
# nan_to_num placement; gdn2_backward_staged composes them as _gdn2_core_bwd.

def dav_backward(Aqk, v_new, do, dtype=torch.float64):
    """Kernel B2, ``dav_backward_pallas`` (kernel_bwd_b2_dav.py:17-51):
    dAqk = nan_to_num((do v_new^T) * causal), dv_new = nan_to_num(Aqk^T do)."""
    f = dtype
    Aqk, v_new, do = (t.to(f) for t in (Aqk, v_new, do))
    BT = Aqk.shape[-1]
    causal = torch.tril(torch.ones(BT, BT, dtype=f))                           # :24
    dAqk = n2n((do @ v_new.transpose(-1, -2)) * causal)                       # :26,29
    dv_new = n2n(Aqk.transpose(-1, -2) @ do)                                  # :27,30
    return dAqk, dv_new


def dhu_backward(do, dv_partial, w_pseudo, qg, kg, gc_last, scale, dht=None, dtype=torch.float64):
    """Kernel B1, ``gdn2_dhu_backward`` (kernel_bwd_b1_dhu.py:14-44): the
    reverse scan over blocks.  Returns ``(dh_all, dh0, dv_all)``: dh_all[:, :, n]
    is the carry after block n, i.e. the gradient of the state entering it."""
    f = dtype
    do, dvp, wp, qg, kg, gcl = (t.to(f) for t in (do, dv_partial, w_pseudo, qg, kg, gc_last))
    B, H, NT, BT, K = qg.shape
    V = do.shape[-1]
    dh = torch.zeros(B, H, K, V, dtype=f) if dht is None else dht.to(f)        # :16-17
    dh = sanitize(dh)                                                         # :18
    dh_all, dv_all = [None] * NT, [None] * NT
    for n in reversed(range(NT)):                                             # :42
        decay = torch.exp(gcl[:, :, n])[..., None]                            # :24
        from_out = qg[:, :, n].transpose(-1, -2) @ (scale * do[:, :, n])      # :26-27
        from_state = dh * decay                                               # :28
        dv_new = sanitize(dvp[:, :, n] + kg[:, :, n] @ dh)                    # :30-32
        from_vnew = -(wp[:, :, n].transpose(-1, -2) @ dv_new)                 # :34
        dh = sanitize(from_out + from_state + from_vnew)                      # :36-37
        dh_all[n], dv_all[n] = dh, dv_new                                     # :39
    return torch.stack(dh_all, 2), dh, torch.stack(dv_all, 2)


def wy_dqkg_backward(q, k, b, w, v, gc, A, Akk, h_pre, v_new, do, dv, dh_next, scale,
                     dtype=torch.float64):
    """Kernel B3, ``wy_dqkg_backward_pallas`` (kernel_bwd_b3_wy_dqkg.py:33-148):
    per block, the gradients through w_pseudo, u, kg, qg and the inverse
    A = (I + Akk)^-1, with dA_total and tmp clipped before the two products
    through A^T (:82-91).  Akk only fixes the shape.  Returns a dict of dq, dk,
    db, dw, dv_raw, dgc (each nan_to_num'd) and dAkk."""
    f = dtype
    q, k, b, w, v, gc, A = (t.to(f) for t in (q, k, b, w, v, gc, A))
    h_pre, v_new, do, dv, dh_next = (t.to(f) for t in (h_pre, v_new, do, dv, dh_next))
    BT = A.shape[-1]
    gcl = gc[..., BT - 1, :]                                                  # :53
    egc = torch.exp(gc)
    kb = b * k * egc                                                          # :55
    ekg = torch.exp(gcl[..., None, :] - gc)
    kg = k * ekg                                                              # :56
    qg = q * egc                                                              # :57
    wv = w * v                                                                # :58
    dqg = (scale * do) @ h_pre.transpose(-1, -2)                              # :60-61
    dw_pseudo = (-dv) @ h_pre.transpose(-1, -2)                               # :63-64
    du = dv                                                                   # :65
    dkg = v_new @ dh_next.transpose(-1, -2)                                   # :67
    dA_from_w = dw_pseudo @ kb.transpose(-1, -2)                              # :69
    dkb = A.transpose(-1, -2) @ dw_pseudo                                     # :70
    dA_from_u = du @ wv.transpose(-1, -2)                                     # :72
    dwv = A.transpose(-1, -2) @ du                                            # :73
    dA_total = sanitize(dA_from_w + dA_from_u)                                # :75,78
    strict = torch.tril(torch.ones(BT, BT, dtype=f), diagonal=-1)             # :80-81
    tmp = sanitize(dA_total @ A.transpose(-1, -2))                            # :83-84
    dAkk = -(A.transpose(-1, -2) @ tmp) * strict                              # :85-86
    dk_from_kb = dkb * egc * b                                                # :88
    db_ = dkb * egc * k                                                       # :89
    dgc_from_kb = dkb * kb                                                    # :90
    dx = dkg * kg                                                             # :92
    dk_from_kg = dkg * ekg                                                    # :93
    dgc_last_contrib = dx.sum(-2)                                             # :95
    dq = dqg * egc                                                            # :97
    dgc_from_qg = dqg * qg                                                    # :98
    dw_ = dwv * v                                                             # :100
    dv_raw = dwv * w                                                          # :101
    dk = dk_from_kb + dk_from_kg                                              # :103
    dgc = dgc_from_kb + dgc_from_qg - dx                                      # :94,104
    dgc_last_from_decay = torch.exp(gcl) * (dh_next * h_pre).sum(-1)          # :106-107
    dgc = dgc.clone()
    dgc[..., BT - 1, :] = dgc[..., BT - 1, :] + dgc_last_contrib + dgc_last_from_decay   # :108-111
    return dict(dq=n2n(dq), dk=n2n(dk), db=n2n(db_), dw=n2n(dw_), dv_raw=n2n(dv_raw),
                dgc=n2n(dgc), dAkk=n2n(dAkk))                                 # :113-119


def intra_backward(dAqk, dAkk, q, k, b, g, scale, sub=128, dtype=torch.float64):
    """Kernel B4, ``intra_backward_pallas`` (kernel_bwd_b4_intra.py:57-165):
    the backward of kernel A over its ``sub``-row sub-block pairs (si >= sj),
    pairwise exp(clip(gc_i - gc_j, +-20)) with the clip mask on the dgc terms,
    causal / strict masks on diagonal sub-blocks, and a clip to +-1e4 after
    every accumulation (:113-121).  q, k, b, g [B, T, H, D]; dAqk, dAkk
    [B, H, NT, BT, BT].  Returns dq, dk, db, dgc [B, H, NT, BT, D]."""
    f = dtype
    BT = dAqk.shape[-1]
    q_, k_, b_, g_ = (_blocks(t.to(f), BT) for t in (q, k, b, g))
    dAqk, dAkk = dAqk.to(f), dAkk.to(f)
    gc = torch.cumsum(g_, dim=-2)                                              # :66-68
    bk = b_ * k_                                                               # :70
    dq = torch.zeros_like(q_)
    dk = torch.zeros_like(q_)
    dbk = torch.zeros_like(q_)
    dgc = torch.zeros_like(q_)
    idx = torch.arange(sub)
    causal = (idx[:, None] >= idx[None, :]).to(f)
    strict = (idx[:, None] > idx[None, :]).to(f)
    for si in range(BT // sub):                                                # :77-78
        for sj in range(si + 1):
            i0, j0 = si * sub, sj * sub
            I, J = slice(i0, i0 + sub), slice(j0, j0 + sub)
            dd = gc[..., I, None, :] - gc[..., None, J, :]                      # :89
            cm = ((dd >= -CLIP_DECAY) & (dd <= CLIP_DECAY)).to(f)               # :90
            e = torch.exp(torch.clamp(dd, -CLIP_DECAY, CLIP_DECAY))             # :91
            mqk, mkk = dAqk[..., I, J], dAkk[..., I, J]
            if si == sj:                                                      # :95-99
                mqk, mkk = mqk * causal, mkk * strict
            Lqk, Rk, Lkk = scale * q_[..., I, :], k_[..., J, :], bk[..., I, :]
            wq = mqk[..., None] * e                                           # dM * edecay
            wk = mkk[..., None] * e
            dL_qk = (wq * Rk[..., None, :, :]).sum(-2)                        # :38-41,103
            dR_qk = (wq * Lqk[..., :, None, :]).sum(-3)                       # :44-47,104
            gq = wq * Lqk[..., :, None, :] * Rk[..., None, :, :] * cm          # :50-54,105
            dL_kk = (wk * Rk[..., None, :, :]).sum(-2)                        # :109
            dR_kk = (wk * Lkk[..., :, None, :]).sum(-3)                       # :110
            gk = wk * Lkk[..., :, None, :] * Rk[..., None, :, :] * cm          # :111
            dq[..., I, :] = sanitize(dq[..., I, :] + dL_qk * scale)            # :117
            dbk[..., I, :] = sanitize(dbk[..., I, :] + dL_kk)                 # :118
            dk[..., J, :] = sanitize(dk[..., J, :] + dR_qk + dR_kk)           # :119
            dgc[..., I, :] = sanitize(dgc[..., I, :] + gq.sum(-2) + gk.sum(-2))      # :120
            dgc[..., J, :] = sanitize(dgc[..., J, :] - gq.sum(-3) - gk.sum(-3))      # :121
    dk_f = dk + dbk * b_                                                       # :124
    db_f = dbk * k_                                                            # :125
    return sanitize(dq), sanitize(dk_f), sanitize(db_f), sanitize(dgc)         # :129-132


def reverse_cumsum_bwd(dgc, chunk_size):
    """Kernel B5, ``reverse_cumsum_bwd`` (kernel_bwd_b5_reverse_cumsum.py:17-24):
    the suffix sum over each block's rows, clipped to +-1e4."""
    return sanitize(torch.flip(torch.cumsum(torch.flip(dgc, [-2]), -2), [-2]))


def _unblocks(t):
    """[B, H, NT, BT, D] -> [B, T, H, D] (_reshape_out, kernel_trainable_B6.py)."""
    B, H, NT, BT, D = t.shape
    return t.permute(0, 2, 3, 1, 4).reshape(B, NT * BT, H, D)


def gdn2_backward_staged(q, k, v, w, b, g, scale, do, dh_final=None, h0=None, block=256,
                         dtype=torch.float64):
    """``_gdn2_core_bwd`` (kernel_trainable_B6.py:97-181) from the stage
    restatements: kernels A, B, C, D-with-state, then B2, B1, B3, B4, B5 and
    the final sanitise.  Drop-in argument order; returns
    ``(dq, dk, dv, dw, db, dg, dh0)``."""
    f = dtype
    B, T, H, K = q.shape
    V = v.shape[-1]
    Aqk, Akk = chunk_scores(q, k, b, g, scale, block=block, dtype=f)
    A = wy_solve_blocked(Akk)
    wp, u, kg, qg, gcl = recompute_wy(q, k, v, w, b, g, A, dtype=f)
    _, _, h_pre, v_new = gdn2_inter_chunk_combine(Aqk, wp, u, kg, qg, gcl, scale, h0=h0, dtype=f,
                                                  return_state=True)
    gc = torch.cumsum(_blocks(g.to(f), block), dim=-2)                          # :116-118
    q_r, k_r, b_r, w_r, v_r, do_r = (_blocks(t.to(f), block) for t in (q, k, b, w, v, do))
    dAqk, dv_partial = dav_backward(Aqk, v_new, do_r, dtype=f)                  # :127
    dht = torch.zeros(B, H, K, V, dtype=f) if dh_final is None else dh_final.to(f)
    dh_all, dh0, dv_all = dhu_backward(do_r, dv_partial, wp, qg, kg, gcl, scale, dht=dht, dtype=f)
    dh_next = torch.cat([dh_all[:, :, 1:], dht[:, :, None]], dim=2)             # :80-83,130
    b3 = wy_dqkg_backward(q_r, k_r, b_r, w_r, v_r, gc, A, Akk, h_pre, v_new, do_r, dv_all, dh_next,
                          scale, dtype=f)
    dq4, dk4, db4, dgc4 = intra_backward(dAqk, b3["dAkk"], q, k, b, g, scale, dtype=f)
    dg = reverse_cumsum_bwd(b3["dgc"] + dgc4, block)                            # :142-143
    outs = (b3["dq"] + dq4, b3["dk"] + dk4, b3["dv_raw"], b3["dw"], b3["db"] + db4, dg)
    return tuple(final_sanitize(_unblocks(t)) for t in outs) + (final_sanitize(dh0),)
