"""Seeded random shapes of the widened rows on the GPU against the CPU
oracle's bf16 dtype flow (tolerance 2e-2, norm-wise per tensor): the output
epilogue (RMSNorm + SiLU gate, both variants) at every row width it takes
with ragged row counts, the GDN2 prologue (batch 1-3, lengths 128-384, head
sizes 64 / 128, model widths 512-2560) and the Mamba2 prologue with its
projections (state sizes 64-256, so the projection GEMM's width d + 2N ends
in partial tiles)."""
import random

import pytest
import torch

from _util import TOL_BF16, banner, rel_err
from atomic_ops import norm_gate as NG
from atomic_ops import prologue as PL
from oracle import norm_gate as ong
from oracle import prologue as op

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _check(errs):
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < TOL_BF16, (k, v)


def _cases(seed):
    rng = random.Random(seed)
    out = []
    for m in (1, 2, 3, 4, 6, 8, 12, 16):   # the instantiated widths, 512 m
        for v in ("gdn2", "mamba2"):
            out.append(("norm_gate", (v, rng.choice([1, 3, 17, 255, 257, 513, 1030]), 512 * m,
                                      rng.choice([1.0, 3.0, 60.0]), rng.randrange(1000))))
    for _ in range(8):
        dh = rng.choice([64, 128]); d = 512 * rng.choice([1, 2, 3, 4, 5])
        out.append(("prologue", (rng.choice([1, 2, 3]), 128 * rng.choice([1, 2, 3]), d // dh, dh, rng.randrange(1000))))
    for _ in range(8):
        P = rng.choice([64, 128]); d = 512 * rng.choice([1, 2, 3, 4, 5, 6])
        out.append(("proj", (rng.choice([1, 2, 3]), 128 * rng.choice([1, 2, 3]), d // P, P, 64 * rng.choice([1, 2, 3, 4]),
                             rng.randrange(1000))))
    return out


CASES = _cases(5)


def _norm_gate(v, rows, d, gs, seed):
    variant, ovar = (NG.GDN2, ong.GDN2) if v == "gdn2" else (NG.MAMBA2, ong.MAMBA2)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, d, generator=g) * (40.0 if v == "mamba2" else 1.0)
    gate = (gs * torch.randn(rows, d, generator=g)).to(BF16)
    w = 1.0 + 0.2 * torch.randn(d, generator=g)
    dout = torch.randn(rows, d, generator=g).to(BF16)
    out_ref = ong.out_norm_gate(x, gate, w, ovar)
    dx_ref, dg_ref, dw_ref = ong.out_norm_gate_grads(x, gate, w, dout, ovar)
    xc, gc, wc = x.cuda(), gate.cuda(), w.cuda()
    out = NG.forward(xc, gc, wc, variant)
    dx, dg, dw = NG.backward(xc, gc, wc, dout.cuda(), variant)
    torch.cuda.synchronize()
    _check({"out": rel_err(out, out_ref), "dx": rel_err(dx, dx_ref), "dgate": rel_err(dg, dg_ref),
            "dweight": rel_err(dw, dw_ref)})


def _prologue(B, L, H, dh, seed):
    g = torch.Generator().manual_seed(seed)
    d = H * dh
    r = lambda *s: torch.randn(*s, generator=g)
    ins = [r(B, L, d).to(BF16) for _ in range(3)] + [0.5 * r(3, d, 4), 0.1 * r(3, d)]
    ins += [r(B, L, d).to(BF16), r(B, L, d).to(BF16), (r(B, L, d) + 1.0).to(BF16), r(H)]
    cots = [r(B, L, H, dh).to(BF16) for _ in range(5)] + [r(B, L, H, dh)]
    ref_out = op.gdn2_prologue(*ins, H)
    ref_grads = op.gdn2_prologue_grads(ins, cots, H)
    gi = [t.cuda() for t in ins]
    outs = PL.forward(*gi, H)
    grads = PL.backward(*gi, H, *(c.cuda() for c in cots))
    torch.cuda.synchronize()
    errs = {n: rel_err(a, b) for n, a, b in zip(("q", "k", "v", "w", "b", "g"), outs, ref_out)}
    errs.update({n: rel_err(a, b) for n, a, b in zip(
        ("dq_lin", "dk_lin", "dv_lin", "dconv_w", "dconv_b", "db_pre", "dw_pre", "df_pre", "da"), grads, ref_grads)})
    _check(errs)


def _proj(B, L, H, P, N, seed):
    g = torch.Generator().manual_seed(seed)
    d = H * P
    r = lambda *s: torch.randn(*s, generator=g)
    in_proj = r(B, L, 2 * d).to(BF16)
    params = [0.5 * r(d, 4), 0.1 * r(d), r(d, d) / d ** 0.5, r(d) - 2.0, r(d, N) / d ** 0.5, r(d, N) / d ** 0.5,
              r(H)]
    cots = [r(B, L, H, P).to(BF16), r(B, L, H, P).to(BF16), r(B, L, N).to(BF16), r(B, L, N).to(BF16), r(H)]
    x_bc = in_proj[..., :d]
    ref_out = op.mamba2_proj_prologue(x_bc, *params, H)
    ref_pre = op.mamba2_projections(x_bc, *params[2:6])
    ref_grads = op.mamba2_proj_prologue_grads([x_bc] + params, cots, H)
    gp = in_proj.cuda()
    gparams = [t.cuda() for t in params]
    outs, pres = PL.mamba2_proj_forward(gp[..., :d], *gparams, H, save=True)
    d_in = torch.full_like(gp, 7.0)
    grads = PL.mamba2_proj_backward(gp[..., :d], *gparams, H, pres, *(c.cuda() for c in cots), dx_bc=d_in)
    torch.cuda.synchronize()
    errs = {}
    for names, got, ref in ((("x", "dt", "B", "C", "A"), outs, ref_out), (("dt_pre", "b_pre", "c_pre"), pres, ref_pre),
                            (("dx_bc", "dconv_w", "dconv_b", "dw_dt", "db_dt", "dw_b", "dw_c", "da_log"), grads,
                             ref_grads)):
        for n, a, b in zip(names, got, ref):
            assert a.shape == b.shape and a.dtype == b.dtype, n
            errs[n] = rel_err(a, b)
    # the gradient lands in the x_bc half of the in_proj gradient only
    assert torch.equal(d_in[..., d:].cpu(), torch.full((B, L, d), 7.0, dtype=BF16))
    _check(errs)


def _name(c):
    kind, a = c
    return kind + "-" + "-".join(str(v) for v in a)


@pytest.mark.parametrize("case", CASES, ids=[_name(c) for c in CASES])
def test_random_shapes_of_the_widened_rows(case):
    kind, args = case
    banner(_name(case))
    {"norm_gate": _norm_gate, "prologue": _prologue, "proj": _proj}[kind](*args)
