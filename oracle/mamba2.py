"""Mamba2 SSD chunk-scan oracle: CPU restatement of the reference.

Test infrastructure only (see ``oracle/__init__.py``).

Conventions (reference ``atomic_ops/mamba2_ssd_reference.py:152-179``):
  dt, x : [B, T, H, P]   (dt is per head *and* channel, model.py:427,471)
  A     : [H]            (negative log-decay rate per unit dt)
  Bm, Cm: [B, T, N]      (shared by every head, ngroups = 1)
  state : [B, H, P, N]   fp32 carry
  y     : [B, T, H, P]   fp32 (mamba2_ssd_reference.py:148,178)
There is no ``D * x`` skip term in the reference (it takes no D argument,
mamba2_ssd_reference.py:152).
"""
from __future__ import annotations

import torch

CLIP_STEP = 20.0
CLIP_ACC = 1e4


def sanitize(x, c=CLIP_ACC):
    """``_sanitize`` (mamba2_ssd_reference.py:66-67)."""
    return torch.nan_to_num(torch.clamp(x, -c, c), nan=0.0, posinf=c, neginf=-c)


def clip_mask(x, lo, hi):
    """Straight-through mask of ``clip`` (mamba2_bwd_reference.py:48-52)."""
    return ((x >= lo) & (x <= hi)).to(x.dtype)


def chunk_ssd(dt_c, A, B_c, C_c, x_c, state_prev, dtype=torch.float64):
    """One chunk of the SSD forward (mamba2_ssd_reference.py:70-149).

    Layout: dt_c, x_c [b, C, h, p]; B_c, C_c [b, C, n]; state_prev [b, h, p, n].
    Returns ``(y_c, state_new, parts)``; ``parts`` holds the intermediates
    the kernel-level tests check (cumdecay, y_diag, state_end, y_off)."""
    f = dtype
    Cs = dt_c.shape[1]
    dA_exponent = sanitize(torch.einsum("bchd,h->bchd", dt_c.to(f), A.to(f)), CLIP_STEP)  # :85-86
    idx = torch.arange(Cs)
    tril_ones = (idx[:, None] >= idx[None, :]).to(f)
    cumdecay = torch.einsum("ij,bjhd->bihd", tril_ones, dA_exponent)                 # :98-100
    cumdecay = sanitize(cumdecay, CLIP_ACC)                                           # :115
    decay_diff = cumdecay[:, :, None] - cumdecay[:, None, :]                          # :117
    causal = (idx[:, None] >= idx[None, :]).to(f)[None, :, :, None, None]             # :118
    L = torch.exp(torch.clamp(decay_diff, -CLIP_STEP, CLIP_STEP)) * causal            # :119
    L = sanitize(L, 1e6)                                                              # :120
    BC_inner = sanitize(torch.einsum("bis,bjs->bij", C_c.to(f), B_c.to(f)))         # :122-123
    dBx = sanitize(dt_c.to(f) * x_c.to(f))                                            # :125-126
    weight = L * BC_inner[:, :, :, None, None]                                        # :129
    y_diag = sanitize(torch.einsum("bijhd,bjhd->bihd", weight, dBx))                  # :130-131
    decay_to_end = torch.exp(torch.clamp(cumdecay[:, -1:] - cumdecay, -CLIP_STEP, CLIP_STEP))  # :133
    decay_to_end = sanitize(decay_to_end, 1e6)                                        # :134
    write = dBx * decay_to_end                                                        # :135
    state_end = sanitize(torch.einsum("bcs,bchd->bhds", B_c.to(f), write))            # :136-137
    decay_h = torch.exp(torch.clamp(cumdecay, -CLIP_STEP, 0.0))                       # :139
    y_off = sanitize(torch.einsum("bis,bhds->bihd", C_c.to(f), state_prev) * decay_h)  # :140-142
    decay_chunk_end = torch.exp(torch.clamp(cumdecay[:, -1], -CLIP_STEP, 0.0))        # :144
    state_new = sanitize(state_prev * decay_chunk_end[..., None] + state_end)         # :145-146
    y_c = sanitize(y_diag + y_off)                                                    # :148
    parts = dict(cumdecay=cumdecay, y_diag=y_diag, state_end=state_end, y_off=y_off,
                 CB=BC_inner)
    return y_c, state_new, parts


def _to_chunks(t, C):
    """[b, l, ...] -> [n_chunks, b, C, ...] (mamba2_ssd_reference.py:161-164)."""
    b, l = t.shape[:2]
    return t.reshape(b, l // C, C, *t.shape[2:]).transpose(0, 1)


def _from_chunks(t):
    """[n_chunks, b, C, ...] -> [b, l, ...] (mamba2_bwd_reference.py:249-257)."""
    t = t.transpose(0, 1)
    return t.reshape(t.shape[0], t.shape[1] * t.shape[2], *t.shape[3:])


def mamba2_ssd_reference(dt, A, Bm, Cm, x, chunk_size, state0=None, dtype=torch.float64,
                         return_parts=False):
    """Chunked SSD forward (mamba2_ssd_reference.py:152-179).  Argument
    order follows the reference function ``(dt, A, B, C, x, ...)``."""
    f = dtype
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    assert l % chunk_size == 0                                                        # :158
    state = torch.zeros(b, h, p, n, dtype=f) if state0 is None else state0.to(f)     # :168-169
    dtc, Bc, Cc, xc = (_to_chunks(t, chunk_size) for t in (dt, Bm, Cm, x))
    ys, parts = [], []
    for c in range(l // chunk_size):
        y_c, state, pr = chunk_ssd(dtc[c], A, Bc[c], Cc[c], xc[c], state, dtype=f)
        ys.append(y_c)
        parts.append(pr)
    y = _from_chunks(torch.stack(ys, 0))
    if return_parts:
        return y, state, parts
    return y, state


def mamba2_token_serial(dt, A, Bm, Cm, x, state0=None, dtype=torch.float64):
    """Token-serial SSM ``s_t = exp(dt_t A) s_{t-1} + (dt_t x_t) B_t^T``,
    ``y_t = s_t C_t`` -- the recurrence the chunked form decomposes
    (mamba2_ssd_reference.py:14-29).  No clipping, so it agrees with the
    chunked form only while no clip fires."""
    f = dtype
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    s = torch.zeros(b, h, p, n, dtype=f) if state0 is None else state0.to(f)
    ys = []
    for t in range(l):
        dtt = dt[:, t].to(f)
        decay = torch.exp(dtt * A.to(f)[None, :, None])
        s = s * decay[..., None] + (dtt * x[:, t].to(f))[..., None] * Bm[:, t].to(f)[:, None, None, :]
        ys.append(torch.einsum("bhpn,bn->bhp", s, Cm[:, t].to(f)))
    return torch.stack(ys, 1), s


# ---------------------------------------------------------------- stages
# The staged forward the reference's trainable wrapper runs
# (mamba2_pallas_forward, kernel_mamba2_c_interchunk.py:90-100): M2 -> M3 ->
# M4 over per-chunk arrays [b, h, NT, C, p] (cumdecay) and [b, h, NT, p, n]
# (state_end).  Same mathematics as mamba2_ssd_reference; the stage kernels
# drop the 1e6 caps on the pair weight and the decay to the chunk end,
# sanitise the chunk's write, accumulate y_diag per 128-row sub-block
# (sanitising between them) and sanitise state0.

def _stage_chunks(t, C):
    """[b, l, h, d] -> [b, h, NT, C, d]."""
    b, l, h, d = t.shape
    return t.reshape(b, l // C, C, h, d).permute(0, 3, 1, 2, 4)


def _stage_unchunk(t):
    """[b, h, NT, C, d] -> [b, l, h, d]."""
    b, h, nt, C, d = t.shape
    return t.permute(0, 2, 3, 1, 4).reshape(b, nt * C, h, d)


def build_chunk_cumdecay(dt, A, chunk_size, dtype=torch.float64):
    """M2 (kernel_mamba2_a_decay.py:53-66): per chunk,
    sanitize(tril @ sanitize(dt A, 20), 1e4) -> [b, h, NT, C, p]."""
    f = dtype
    dA = sanitize(dt.to(f) * A.to(f)[None, None, :, None], CLIP_STEP)              # :59-60
    cum = torch.cumsum(_stage_chunks(dA, chunk_size), dim=3)                     # :62-64 (tril @ dA)
    return sanitize(cum, CLIP_ACC)                                              # :66


def intra_chunk_ssd(dt, x, Bm, Cm, cumdecay, chunk_size, dtype=torch.float64):
    """M3 (kernel_mamba2_b_intra.py:69-116): (y_diag [b, l, h, p],
    state_end [b, h, NT, p, n])."""
    f = dtype
    C = chunk_size
    bc = min(128, C)                                                            # :61-62,71
    dtc, xc = (_stage_chunks(t.to(f), C) for t in (dt, x))                      # [b, h, nt, C, p]
    b, h, nt = dtc.shape[:3]
    Bc = Bm.to(f).reshape(b, nt, C, -1)[:, None]                                # broadcast over heads (:137-142)
    Cc = Cm.to(f).reshape(b, nt, C, -1)[:, None]
    cum = cumdecay.to(f)
    dBx = sanitize(dtc * xc)                                                    # :81
    BC_inner = sanitize(Cc @ Bc.transpose(-1, -2))                              # :83-84
    y_diag = torch.zeros_like(dtc)                                              # :86
    idx = torch.arange(bc)
    causal = (idx[:, None] >= idx[None, :]).to(f)
    for si in range(C // bc):                                                   # :88-108
        for sj in range(si + 1):
            i0, j0 = si * bc, sj * bc
            dd = cum[..., i0:i0 + bc, None, :] - cum[..., None, j0:j0 + bc, :]
            w = torch.exp(torch.clamp(dd, -CLIP_STEP, CLIP_STEP)) * BC_inner[..., i0:i0 + bc, j0:j0 + bc, None]
            if si == sj:
                w = w * causal[:, :, None]
            y_blk = torch.einsum("...ijd,...jd->...id", w, dBx[..., j0:j0 + bc, :])
            y_diag[..., i0:i0 + bc, :] = sanitize(y_diag[..., i0:i0 + bc, :] + y_blk)
    dte = torch.exp(torch.clamp(cum[..., -1:, :] - cum, -CLIP_STEP, CLIP_STEP))  # :111-112
    write = sanitize(dBx * dte)                                                 # :113
    state_end = sanitize(torch.einsum("...jd,...js->...ds", write, Bc.expand(-1, h, -1, -1, -1)))  # :115-116
    return _stage_unchunk(y_diag), state_end


def mamba2_inter_chunk_combine(y_diag, state_end, cumdecay, Cm, chunk_size, state0=None, dtype=torch.float64):
    """M4 (kernel_mamba2_c_interchunk.py:38-87): (y [b, l, h, p],
    state_final [b, h, p, n])."""
    f = dtype
    C = chunk_size
    b, l, h, p = y_diag.shape
    n = Cm.shape[-1]
    nt = l // C
    ydc = _stage_chunks(y_diag.to(f), C)
    Cc = Cm.to(f).reshape(b, nt, C, n)
    state = torch.zeros(b, h, p, n, dtype=f) if state0 is None else state0.to(f)
    state = sanitize(state)                                                     # :58
    ys = []
    for c in range(nt):                                                         # :68-80
        cum = cumdecay[:, :, c].to(f)                                           # [b, h, C, p]
        dfs = torch.exp(torch.clamp(cum, -CLIP_STEP, 0.0))
        y_off = sanitize(torch.einsum("bis,bhds->bhid", Cc[:, c], state) * dfs)
        dce = torch.exp(torch.clamp(cum[:, :, -1, :], -CLIP_STEP, 0.0))
        state = sanitize(state * dce[..., None] + state_end[:, :, c].to(f))
        ys.append(sanitize(ydc[:, :, c] + y_off))
    return _stage_unchunk(torch.stack(ys, 2)), state


def intra_chunk_ssd_loops(dt, x, Bm, Cm, cumdecay, chunk_size):
    """M3 element by element in Python floats (tiny inputs only): the
    independent restatement the vectorised one is checked against."""
    import math
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    C = chunk_size
    bc = min(128, C)
    cl = lambda v, c: 0.0 if math.isnan(v) else min(max(v, -c), c)
    y = torch.zeros(b, l, h, p, dtype=torch.float64)
    se = torch.zeros(b, h, l // C, p, n, dtype=torch.float64)
    for bb in range(b):
        for c in range(l // C):
            t0 = c * C
            cb = [[cl(sum(float(Cm[bb, t0 + i, s]) * float(Bm[bb, t0 + j, s]) for s in range(n)), CLIP_ACC)
                   for j in range(C)] for i in range(C)]
            for hh in range(h):
                for d in range(p):
                    cum = [float(cumdecay[bb, hh, c, i, d]) for i in range(C)]
                    dbx = [cl(float(dt[bb, t0 + j, hh, d]) * float(x[bb, t0 + j, hh, d]), CLIP_ACC) for j in range(C)]
                    for i in range(C):
                        acc = 0.0
                        for sj in range(i // bc + 1):
                            blk = 0.0
                            for j in range(sj * bc, min((sj + 1) * bc, i + 1)):
                                blk += math.exp(cl(cum[i] - cum[j], CLIP_STEP)) * cb[i][j] * dbx[j]
                            acc = cl(acc + blk, CLIP_ACC)
                        y[bb, t0 + i, hh, d] = acc
                    for s in range(n):
                        v = sum(cl(dbx[j] * math.exp(cl(cum[-1] - cum[j], CLIP_STEP)), CLIP_ACC) * float(Bm[bb, t0 + j, s])
                                for j in range(C))
                        se[bb, hh, c, d, s] = cl(v, CLIP_ACC)
    return y, se


def chunk_ssd_bwd(dt_c, A, B_c, C_c, x_c, state_prev, dy_c, dstate_new, dtype=torch.float64, cb_round=None):
    """Hand-derived backward of one chunk: MB0 ``_chunk_ssd_bwd``
    (mamba2_bwd_reference.py:55-197).  Returns
    ``(ddt_c, dB_c, dC_c, dx_c, dA, dstate_prev, dcum_total)``; the last one
    (the combined cumdecay cotangent after the last-row terms) is exposed for
    kernel-level tests.  ``cb_round`` (a torch dtype; tests only) rounds the
    C.B^T scores to that type, which emulates a kernel that stages them at
    that precision; the reference keeps them float32."""
    f = dtype
    dt_c, B_c, C_c, x_c, state_prev = (t.to(f) for t in (dt_c, B_c, C_c, x_c, state_prev))
    dy_c = dy_c.to(f)
    dstate_new = dstate_new.to(f)
    A = A.to(f)
    Cs = dt_c.shape[1]
    # forward re-run (:76-108)
    dA_exponent_raw = torch.einsum("bchd,h->bchd", dt_c, A)
    dA_exponent = sanitize(dA_exponent_raw, CLIP_STEP)
    idx = torch.arange(Cs)
    tril_ones = (idx[:, None] >= idx[None, :]).to(f)
    cumdecay_raw = torch.einsum("ij,bjhd->bihd", tril_ones, dA_exponent)
    cumdecay = sanitize(cumdecay_raw, CLIP_ACC)
    decay_diff_raw = cumdecay[:, :, None] - cumdecay[:, None, :]
    causal = (idx[:, None] >= idx[None, :]).to(f)[None, :, :, None, None]
    L = sanitize(torch.exp(torch.clamp(decay_diff_raw, -CLIP_STEP, CLIP_STEP)) * causal, 1e6)
    BC_inner = sanitize(torch.einsum("bis,bjs->bij", C_c, B_c))
    if cb_round is not None:
        BC_inner = BC_inner.to(cb_round).to(f)
    dBx = sanitize(dt_c * x_c)
    weight = L * BC_inner[:, :, :, None, None]
    decay_to_end_raw = cumdecay[:, -1:] - cumdecay
    decay_to_end = sanitize(torch.exp(torch.clamp(decay_to_end_raw, -CLIP_STEP, CLIP_STEP)), 1e6)
    write = sanitize(dBx * decay_to_end)
    decay_h = torch.exp(torch.clamp(cumdecay, -CLIP_STEP, 0.0))
    y_off_raw = torch.einsum("bis,bhds->bihd", C_c, state_prev)
    decay_chunk_end = torch.exp(torch.clamp(cumdecay[:, -1], -CLIP_STEP, 0.0))
    # reverse pass (:111-197)
    dy_diag = dy_c
    dy_off = dy_c
    dstate_prev = dstate_new * decay_chunk_end[..., None]                              # :115
    d_decay_chunk_end = (dstate_new * state_prev).sum(-1)                              # :116
    dstate_end = dstate_new
    d_cum_last_a = d_decay_chunk_end * decay_chunk_end * clip_mask(cumdecay[:, -1], -CLIP_STEP, 0.0)  # :120
    dy_off_raw = dy_off * decay_h                                                      # :123
    d_decay_h = dy_off * y_off_raw                                                     # :126
    dC_1 = torch.einsum("bihd,bhds->bis", dy_off_raw, state_prev)                      # :127
    dstate_prev = dstate_prev + torch.einsum("bihd,bis->bhds", dy_off_raw, C_c)        # :128
    d_cum_from_yoff = d_decay_h * decay_h * clip_mask(cumdecay, -CLIP_STEP, 0.0)       # :131
    dwrite = torch.einsum("bhds,bcs->bchd", dstate_end, B_c)                           # :134
    dB_1 = torch.einsum("bhds,bchd->bcs", dstate_end, write)                           # :135
    d_dBx_1 = dwrite * decay_to_end                                                    # :138
    d_decay_to_end = dwrite * dBx                                                      # :139
    d_dte_diff = d_decay_to_end * decay_to_end * clip_mask(decay_to_end_raw, -CLIP_STEP, CLIP_STEP)  # :142
    d_cum_last_b = d_dte_diff.sum(1)                                                   # :143
    d_cum_from_dte = -d_dte_diff                                                       # :144
    dweight = torch.einsum("bihd,bjhd->bijhd", dy_diag, dBx)                           # :147
    d_dBx_2 = torch.einsum("bijhd,bihd->bjhd", weight, dy_diag)                        # :148
    dL = dweight * BC_inner[:, :, :, None, None]                                       # :151
    dBC_inner = (dweight * L).sum((-2, -1))                                            # :152
    dC_2 = torch.einsum("bij,bjs->bis", dBC_inner, B_c)                                # :155
    dB_2 = torch.einsum("bij,bis->bjs", dBC_inner, C_c)                                # :156
    d_decay_diff = dL * L * clip_mask(decay_diff_raw, -CLIP_STEP, CLIP_STEP)           # :159
    d_cum_i = d_decay_diff.sum(2)                                                      # :162
    d_cum_j = -d_decay_diff.sum(1)                                                     # :163
    d_dBx_total = sanitize(d_dBx_1 + d_dBx_2)                                          # :166
    ddt_1 = d_dBx_total * x_c                                                          # :167
    dx_c = d_dBx_total * dt_c                                                          # :168
    d_cum_total = sanitize(d_cum_i + d_cum_j + d_cum_from_yoff + d_cum_from_dte)       # :171-173
    row_mask = (idx == (Cs - 1)).to(f)[None, :, None, None]                            # :176
    d_cum_total = d_cum_total + row_mask * (d_cum_last_a + d_cum_last_b)[:, None]      # :177
    d_cum_total = d_cum_total * clip_mask(cumdecay_raw, -CLIP_ACC, CLIP_ACC)           # :181
    triu_ones = (idx[:, None] <= idx[None, :]).to(f)
    d_dA_exp = torch.einsum("ij,bjhd->bihd", triu_ones, d_cum_total)                   # :183
    d_dA_exp = d_dA_exp * clip_mask(dA_exponent_raw, -CLIP_STEP, CLIP_STEP)            # :186
    ddt_2 = torch.einsum("bchd,h->bchd", d_dA_exp, A)                                  # :187
    dA = (d_dA_exp * dt_c).sum((0, 1, 3))                                              # :188
    ddt_c = sanitize(ddt_1 + ddt_2)                                                    # :190
    dB_c = sanitize(dB_1 + dB_2)                                                       # :191
    dC_c = sanitize(dC_1 + dC_2)                                                       # :192
    dx_c = sanitize(dx_c)                                                              # :193
    dA = sanitize(dA)                                                                  # :194
    dstate_prev = sanitize(dstate_prev)                                                # :195
    return ddt_c, dB_c, dC_c, dx_c, dA, dstate_prev, d_cum_total


def chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, chunk_size, do, dstate_final=None, state0=None,
                       dtype=torch.float64, cb_round=None):
    """Full-sequence MB0 backward (mamba2_bwd_reference.py:200-266): forward
    re-run for ``state_prev`` per chunk, then a reverse scan.  Returns
    ``(ddt, dB, dC, dx, dA, dstate0)``.  ``cb_round``: see chunk_ssd_bwd."""
    f = dtype
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    state = torch.zeros(b, h, p, n, dtype=f) if state0 is None else state0.to(f)
    dtc, Bc, Cc, xc, doc = (_to_chunks(t, chunk_size) for t in (dt, Bm, Cm, x, do))
    nc = l // chunk_size
    prevs = []
    for c in range(nc):                                                               # :229-234
        prevs.append(state)
        _, state, _ = chunk_ssd(dtc[c], A, Bc[c], Cc[c], xc[c], state, dtype=f)
    dstate = torch.zeros(b, h, p, n, dtype=f) if dstate_final is None else dstate_final.to(f)
    outs = [None] * nc
    dA = torch.zeros(h, dtype=f)
    for c in reversed(range(nc)):                                                     # :236-247
        ddt_c, dB_c, dC_c, dx_c, dA_c, dstate, _ = chunk_ssd_bwd(
            dtc[c], A, Bc[c], Cc[c], xc[c], prevs[c], doc[c], dstate, dtype=f, cb_round=cb_round)
        outs[c] = (ddt_c, dB_c, dC_c, dx_c)
        dA = dA + dA_c                                                                # :263
    ddt, dB, dC, dx = (_from_chunks(torch.stack([o[i] for o in outs], 0)) for i in range(4))
    return ddt, dB, dC, dx, dA, sanitize(dstate)                                      # :264


def final_sanitize(x):
    """``_final_sanitize`` at the custom_vjp boundary (kernel_mamba2_trainable_B6.py:67-69)."""
    return sanitize(x, CLIP_ACC)


def intra_chunk_ssd_bwd(dt, x, Bm, Cm, cumdecay, dy, dstate_end_grad, chunk_size, dtype=torch.float64):
    """MB2, ``intra_chunk_ssd_bwd_pallas`` (kernel_mamba2_bwd_b2_intra.py:32-180):
    the backward of M3 (y_diag, state_end) per (batch, head, chunk), with the
    state-end part as full-chunk products (:53-66), the y_diag part over
    ``min(128, C)``-row sub-block pairs with a sanitise after every
    accumulation (:74-113), and dB / dC summed over the heads after the
    per-head sanitised values (:168-178).  dt, x, dy [b, l, h, p]; Bm, Cm
    [b, l, n]; cumdecay [b, h, NT, C, p]; dstate_end_grad [b, h, NT, p, n].
    Returns ``(ddt [b, l, h, p], dx [b, l, h, p], dB [b, l, n], dC [b, l, n],
    dcum [b, h, NT, C, p])``."""
    f = dtype
    C = chunk_size
    bc = min(128, C)                                                            # :20-21,35
    dtc, xc, dyc = (_stage_chunks(t.to(f), C) for t in (dt, x, dy))            # [b, h, nt, C, p]
    b, h, nt = dtc.shape[:3]
    n = Bm.shape[-1]
    Bc = Bm.to(f).reshape(b, nt, C, n)[:, None].expand(b, h, nt, C, n)          # :145-148
    Cc = Cm.to(f).reshape(b, nt, C, n)[:, None].expand(b, h, nt, C, n)
    cum = cumdecay.to(f)
    dse = dstate_end_grad.to(f)                                                 # [b, h, nt, p, n]
    dBx = sanitize(dtc * xc)                                                    # :47
    BC_inner = sanitize(Cc @ Bc.transpose(-1, -2))                              # :48
    cl = cum[..., C - 1:, :]                                                    # :50
    dte_raw = cl - cum                                                          # :51
    dte = torch.exp(torch.clamp(dte_raw, -CLIP_STEP, CLIP_STEP))                # :52
    write = sanitize(dBx * dte)                                                 # :53
    dwrite = sanitize(Bc @ dse.transpose(-1, -2))                               # :56  (C, p)
    dB = sanitize(write @ dse)                                                  # :57  (C, n)
    d_dBx_1 = sanitize(dwrite * dte)                                            # :59
    d_dte = sanitize(dwrite * dBx)                                              # :60
    d_dte_diff = sanitize(d_dte * dte * clip_mask(dte_raw, -CLIP_STEP, CLIP_STEP))   # :61-63
    dcum_from_dte = -d_dte_diff                                                 # :64
    dcum_last_b = d_dte_diff.sum(-2)                                            # :65
    d_dBx_2 = torch.zeros_like(dtc)                                             # :68
    dC = torch.zeros_like(Bc)                                                   # :70
    dcum = torch.zeros_like(dtc)                                                # :71
    idx = torch.arange(bc)
    causal = (idx[:, None] >= idx[None, :]).to(f)
    for si in range(C // bc):                                                   # :73-74
        for sj in range(si + 1):
            I, J = slice(si * bc, (si + 1) * bc), slice(sj * bc, (sj + 1) * bc)
            dd = cum[..., I, None, :] - cum[..., None, J, :]                    # :80
            e = torch.exp(torch.clamp(dd, -CLIP_STEP, CLIP_STEP))               # :81
            blk = BC_inner[..., I, J]
            if si == sj:                                                      # :84-87
                blk = blk * causal
            weight = e * blk[..., None]                                       # :89
            dy_i, dbx_j = dyc[..., I, :], dBx[..., J, :]
            dweight = dy_i[..., :, None, :] * dbx_j[..., None, :, :]           # :94
            d_dBx_2_blk = torch.einsum("...ijd,...id->...jd", weight, dy_i)   # :95
            dedecay = dweight * blk[..., None]                                # :97
            dBC_blk = (dweight * e).sum(-1)                                   # :98
            if si == sj:                                                      # :99-100
                dBC_blk = dBC_blk * causal
            dC_blk = dBC_blk @ Bc[..., J, :]                                  # :102
            dB_blk = dBC_blk.transpose(-1, -2) @ Cc[..., I, :]                # :103
            ddd = dedecay * e * clip_mask(dd, -CLIP_STEP, CLIP_STEP)          # :105
            d_dBx_2[..., J, :] = sanitize(d_dBx_2[..., J, :] + d_dBx_2_blk)   # :109
            dB[..., J, :] = sanitize(dB[..., J, :] + dB_blk)                  # :110
            dC[..., I, :] = sanitize(dC[..., I, :] + dC_blk)                  # :111
            dcum[..., I, :] = sanitize(dcum[..., I, :] + ddd.sum(-2))         # :106,112
            dcum[..., J, :] = sanitize(dcum[..., J, :] - ddd.sum(-3))         # :107,113
    d_dBx = sanitize(d_dBx_1 + d_dBx_2)                                         # :116
    ddt = sanitize(d_dBx * xc)                                                  # :118,126
    dx = sanitize(d_dBx * dtc)                                                  # :119,127
    dcum = dcum + dcum_from_dte                                                 # :121
    dcum = dcum.clone()
    dcum[..., C - 1, :] = dcum[..., C - 1, :] + dcum_last_b                     # :122-123
    dcum = sanitize(dcum)                                                       # :128
    dB_out = dB.sum(1).reshape(b, nt * C, n)                                    # :176-178
    dC_out = dC.sum(1).reshape(b, nt * C, n)
    return _stage_unchunk(ddt), _stage_unchunk(dx), dB_out, dC_out, dcum


def state_only_bwd(state_prev, C_c, cumdecay_c, dy_off, dstate_carry, dtype=torch.float64):
    """MB1's per-chunk step, ``_state_only_bwd`` (mamba2_bwd_state_reference.py:87-137):
    the adjoint of y_off = (C state_prev^T) e^{clip(cum, -20, 0)} and of the
    carried state_prev e^{clip(cum_last, -20, 0)}.  state_prev [b, h, p, n],
    C_c [b, C, n], cumdecay_c and dy_off [b, C, h, p], dstate_carry [b, h, p, n].
    Returns ``(dC_c [b, C, n], dstate_prev, dcumdecay_state [b, C, h, p])``, each sanitised."""
    f = dtype
    state_prev, C_c, cum, dy_off, carry = (t.to(f) for t in (state_prev, C_c, cumdecay_c, dy_off, dstate_carry))
    Cs = cum.shape[1]
    decay_h_raw = torch.clamp(cum, -CLIP_STEP, 0.0)                                  # :103
    decay_h = torch.exp(decay_h_raw)
    y_off_raw = torch.einsum("bis,bhds->bihd", C_c, state_prev)                      # :105
    dce = torch.exp(torch.clamp(cum[:, -1], -CLIP_STEP, 0.0))                         # :107-108
    dstate_prev = carry * dce[..., None]                                             # :112
    d_dce = (carry * state_prev).sum(-1)                                             # :113
    d_last_a = d_dce * dce * clip_mask(cum[:, -1], -CLIP_STEP, 0.0)                  # :114
    dy_off_raw = dy_off * decay_h                                                    # :117
    d_decay_h = dy_off * y_off_raw                                                   # :118
    dC_c = torch.einsum("bihd,bhds->bis", dy_off_raw, state_prev)                    # :119
    dstate_prev = dstate_prev + torch.einsum("bihd,bis->bhds", dy_off_raw, C_c)      # :120
    d_cum_yoff = d_decay_h * decay_h * clip_mask(decay_h_raw, -CLIP_STEP, 0.0)       # :123
    row = (torch.arange(Cs) == Cs - 1).to(f)[None, :, None, None]                    # :126
    dcum_state = d_cum_yoff + row * d_last_a[:, None]                                # :127
    return sanitize(dC_c), sanitize(dstate_prev), sanitize(dcum_state)               # :129-131


def mamba2_bwd_scan(dt, A, Bm, Cm, x, chunk_size, do, dstate_final=None, state0=None,
                    dtype=torch.float64):
    """MB1 + MB3, ``mamba2_bwd_scan`` (kernel_mamba2_bwd_b1_state.py:132-254):
    M2's cumdecay, the forward re-run of the reference chunk for the state
    entering each chunk, the state-only reverse scan (its carry, sanitised,
    is MB2's dstate_end_grad), MB2, and the sanitised sums.  Returns
    ``(ddt_partial, dB, dC, dx, dstate0, dcumdecay)``; ddt_partial is the
    dBx = dt x part only, and dcumdecay [b, h, NT, C, p] is both halves'."""
    f = dtype
    b, l, h, p = dt.shape
    n = Bm.shape[-1]
    C = chunk_size
    nc = l // C
    state = torch.zeros(b, h, p, n, dtype=f) if state0 is None else state0.to(f)
    state = sanitize(state)                                                          # :168-170
    cum = build_chunk_cumdecay(dt, A, C, dtype=f)                                    # :184 [b, h, nc, C, p]
    dtc, Bc, Cc, xc, doc = (_to_chunks(t, C) for t in (dt, Bm, Cm, x, do))
    prevs = []
    for c in range(nc):                                                              # :190-195
        prevs.append(state)
        _, state, _ = chunk_ssd(dtc[c], A, Bc[c], Cc[c], xc[c], state, dtype=f)
    carry = torch.zeros(b, h, p, n, dtype=f) if dstate_final is None else dstate_final.to(f)
    dC_state = [None] * nc
    dcum_state = [None] * nc
    used = [None] * nc
    for c in reversed(range(nc)):                                                    # :205-218
        carry = sanitize(carry)
        cum_c = cum[:, :, c].permute(0, 2, 1, 3)                                     # [b, C, h, p]
        dC_c, dprev, dcum_c = state_only_bwd(prevs[c], Cc[c], cum_c, doc[c], carry, dtype=f)
        used[c] = carry
        dC_state[c], dcum_state[c] = dC_c, dcum_c
        carry = sanitize(dprev)
    dstate0 = sanitize(carry)                                                        # :219
    dC_s = torch.stack(dC_state, 1).reshape(b, l, n)                                 # :225
    dse = sanitize(torch.stack(used, 2))                                             # :230-231 [b, h, nc, p, n]
    dcum_s = torch.stack(dcum_state, 2).permute(0, 3, 2, 1, 4)                       # :235 [b, h, nc, C, p]
    ddt_i, dx_i, dB_i, dC_i, dcum_i = intra_chunk_ssd_bwd(dt, x, Bm, Cm, cum, do, dse, C, dtype=f)   # :240-243
    dC = sanitize(dC_s + dC_i)                                                       # :249
    dcum = sanitize(dcum_s + dcum_i)                                                 # :250
    return sanitize(ddt_i), sanitize(dB_i), dC, sanitize(dx_i), dstate0, dcum        # :252-256


def mamba2_dA_backward(dt_pallas, A, dcumdecay, chunk_size, dtype=torch.float64):
    """MB4, ``mamba2_dA_backward`` (mamba2_bwd_a_dA_reference.py:60-115): M2's
    adjoint.  dt_pallas, dcumdecay [b, h, NT, C, p]; A [h].  The cumdecay
    cotangent masked by cumdecay's own clip, reverse-cumsummed over the chunk,
    masked by the step exponent's clip: ddt contribution (sanitised, the
    pallas layout) and dA = sum over everything but the head (sanitised)."""
    f = dtype
    dt_f, A_f, dcum = dt_pallas.to(f), A.to(f), dcumdecay.to(f)
    assert dt_f.shape[3] == chunk_size
    raw = dt_f * A_f[None, :, None, None, None]                                      # :89
    clipped = torch.clamp(raw, -CLIP_STEP, CLIP_STEP)                                # :90
    cum_raw = torch.cumsum(clipped, dim=3)                                           # :92-94
    d_cum_raw = dcum * clip_mask(cum_raw, -CLIP_ACC, CLIP_ACC)                       # :98
    d_clipped = torch.flip(torch.cumsum(torch.flip(d_cum_raw, [3]), 3), [3])         # :101-103
    d_raw = d_clipped * clip_mask(raw, -CLIP_STEP, CLIP_STEP)                        # :106
    ddt2 = d_raw * A_f[None, :, None, None, None]                                    # :109
    dA = (d_raw * dt_f).sum((0, 2, 3, 4))                                            # :110
    return sanitize(ddt2), sanitize(dA)                                              # :112-113
