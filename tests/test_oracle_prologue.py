"""The GDN2 prologue oracle (model.py:574-619) pinned on the CPU: autograd
against central finite differences (float64), causality of the convolution,
and closed forms (identity convolution, unit-norm heads, the decay gate)."""
import pytest
import torch

from _util import rel_err
from oracle import prologue as op

F64 = torch.float64


def _inputs(B, L, H, dh, seed, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    d = H * dh
    r = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    ins = [r(B, L, d) for _ in range(3)] + [0.5 * r(3, d, 4), 0.1 * r(3, d)] + [r(B, L, d) for _ in range(3)] + [r(H)]
    act = [0, 1, 2, 5, 6, 7]
    return [t.to(dtype) if i in act else t for i, t in enumerate(ins)]


def test_autograd_matches_finite_differences():
    B, L, H, dh = 1, 5, 2, 3
    ins = _inputs(B, L, H, dh, 0)
    g = torch.Generator().manual_seed(9)
    cots = [torch.randn(B, L, H, dh, generator=g, dtype=F64) for _ in range(6)]
    grads = op.gdn2_prologue_grads(ins, cots, H, exact=True)

    def loss(args):
        return sum((o * c).sum() for o, c in zip(op.gdn2_prologue(*args, H, exact=True), cots))

    h = 1e-6
    for i, t in enumerate(ins):
        fd = torch.zeros_like(t)
        for idx in range(t.numel()):
            e = torch.zeros(t.numel(), dtype=F64)
            e[idx] = h
            e = e.view(t.shape)
            p = list(ins); p[i] = t + e
            m = list(ins); m[i] = t - e
            fd.view(-1)[idx] = (loss(p) - loss(m)) / (2 * h)
        assert rel_err(grads[i], fd) < 1e-6, i


def test_conv_is_causal_and_identity_taps_pass_through():
    B, L, H, dh = 2, 12, 2, 4
    ins = _inputs(B, L, H, dh, 1)
    out = op.gdn2_prologue(*ins, H, exact=True)
    pert = list(ins)
    pert[0] = ins[0].clone()
    pert[0][:, 7] += 1.0
    out2 = op.gdn2_prologue(*pert, H, exact=True)
    assert torch.equal(out[0][:, :7], out2[0][:, :7])        # no effect before t = 7
    assert not torch.equal(out[0][:, 7:11], out2[0][:, 7:11])
    # taps (0, 0, 0, 1), zero bias: q = normalize(silu(q_lin)), every head unit-norm
    ident = list(ins)
    cw = torch.zeros_like(ins[3]); cw[:, :, 3] = 1.0
    ident[3], ident[4] = cw, torch.zeros_like(ins[4])
    q, k, v = op.gdn2_prologue(*ident, H, exact=True)[:3]
    s = torch.nn.functional.silu(ins[0]).view(B, L, H, dh)
    qn = s / torch.sqrt((s * s).sum(-1, keepdim=True) + 1e-12)
    assert rel_err(q, qn) < 1e-12
    assert rel_err((q * q).sum(-1), torch.ones(B, L, H, dtype=F64)) < 1e-9
    assert rel_err(v, torch.nn.functional.silu(ins[2]).clamp(-50, 50).view(B, L, H, dh)) < 1e-12


def test_decay_gate_closed_form_and_clip():
    B, L, H, dh = 1, 4, 2, 2
    ins = _inputs(B, L, H, dh, 2)
    ins[8] = torch.tensor([0.0, 25.0], dtype=F64)     # a = 0 ; a beyond the +-20 clip
    g = op.gdn2_prologue(*ins, H, exact=True)[5]
    f = ins[7].view(B, L, H, dh)
    sp = torch.log1p(torch.exp(f))
    assert rel_err(g[:, :, 0], -sp[:, :, 0]) < 1e-12
    expect = (-torch.exp(torch.tensor(20.0, dtype=F64)) * sp[:, :, 1]).clamp(-1e3, 1e3)
    assert rel_err(g[:, :, 1], expect) < 1e-12
    cots = [torch.zeros(B, L, H, dh, dtype=F64)] * 5 + [torch.ones(B, L, H, dh, dtype=F64)]
    grads = op.gdn2_prologue_grads(ins, cots, H, exact=True)
    assert grads[8][1] == 0                            # a clipped: no gradient
    assert rel_err(grads[8][0:1], (-sp[:, :, 0]).sum().view(1)) < 1e-12


def test_gradient_sanitiser_clips_q_cotangent():
    B, L, H, dh = 1, 6, 2, 4
    ins = _inputs(B, L, H, dh, 3)
    big = [torch.full((B, L, H, dh), 1e5, dtype=F64)] + [torch.zeros(B, L, H, dh, dtype=F64)] * 5
    cap = [torch.full((B, L, H, dh), 1e3, dtype=F64)] + [torch.zeros(B, L, H, dh, dtype=F64)] * 5
    g1 = op.gdn2_prologue_grads(ins, big, H, exact=True)
    g2 = op.gdn2_prologue_grads(ins, cap, H, exact=True)
    assert rel_err(g1[0], g2[0]) < 1e-12


def test_bf16_flow_stays_near_exact():
    B, L, H, dh = 2, 16, 4, 64
    ins = _inputs(B, L, H, dh, 4, dtype=torch.bfloat16)
    ex = op.gdn2_prologue(*[t.double() for t in ins], H, exact=True)
    bf = op.gdn2_prologue(*ins, H)
    for a, b in zip(bf, ex):
        assert rel_err(a, b) < 2e-2


def _m2_inputs(B, L, H, P, N, seed, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    d = H * P
    r = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    ins = [r(B, L, d), 0.5 * r(d, 4), 0.1 * r(d), r(B, L, d) - 1.0, r(B, L, N), r(B, L, N), r(H)]
    return [t.to(dtype) if i in (0, 3, 4, 5) else t for i, t in enumerate(ins)]


def test_mamba2_prologue_autograd_matches_finite_differences():
    B, L, H, P, N = 1, 5, 2, 2, 3
    ins = _m2_inputs(B, L, H, P, N, 5)
    g = torch.Generator().manual_seed(6)
    cots = [torch.randn(B, L, H, P, generator=g, dtype=F64), torch.randn(B, L, H, P, generator=g, dtype=F64),
            torch.randn(B, L, N, generator=g, dtype=F64), torch.randn(B, L, N, generator=g, dtype=F64),
            torch.randn(H, generator=g, dtype=F64)]
    grads = op.mamba2_prologue_grads(ins, cots, H, exact=True)

    def loss(args):
        return sum((o * c).sum() for o, c in zip(op.mamba2_prologue(*args, H, exact=True), cots))

    h = 1e-6
    for i, t in enumerate(ins):
        fd = torch.zeros_like(t)
        for idx in range(t.numel()):
            e = torch.zeros(t.numel(), dtype=F64)
            e[idx] = h
            e = e.view(t.shape)
            p = list(ins); p[i] = t + e
            m = list(ins); m[i] = t - e
            fd.view(-1)[idx] = (loss(p) - loss(m)) / (2 * h)
        assert rel_err(grads[i], fd) < 1e-6, i


def test_mamba2_prologue_closed_forms():
    B, L, H, P, N = 1, 8, 2, 4, 4
    ins = _m2_inputs(B, L, H, P, N, 7)
    ins[6] = torch.tensor([0.0, 30.0], dtype=F64)
    ins[3] = torch.tensor([-50.0, 0.0, 50.0, 2.0], dtype=F64).repeat(B, L, H * P // 4)
    x, dt, Bo, Co, A = op.mamba2_prologue(*ins, H, exact=True)
    assert rel_err(A, torch.tensor([-1.0, -torch.exp(torch.tensor(20.0, dtype=F64))], dtype=F64)) < 1e-12
    sp = torch.log1p(torch.exp(ins[3])).clamp(1e-2, 1.0).view(B, L, H, P)
    assert rel_err(dt, sp) < 1e-12              # softplus(-50) floors at 1e-2, softplus(50) caps at 1
    assert torch.equal(Bo, ins[4]) and torch.equal(Co, ins[5])
    # identity taps: x = silu(x_bc)
    ident = list(ins)
    cw = torch.zeros_like(ins[1]); cw[:, 3] = 1.0
    ident[1], ident[2] = cw, torch.zeros_like(ins[2])
    assert rel_err(op.mamba2_prologue(*ident, H, exact=True)[0],
                   torch.nn.functional.silu(ins[0]).view(B, L, H, P)) < 1e-12


def _m2x_inputs(B, L, H, P, N, seed, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    d = H * P
    r = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    x_bc = r(B, L, d).to(dtype)
    pd = F64 if dtype == F64 else torch.float32   # the model's parameters are float32
    ps = [0.5 * r(d, 4), 0.1 * r(d), r(d, d) / d ** 0.5, r(d) - 1.0, r(d, N) / d ** 0.5, r(d, N) / d ** 0.5, r(H)]
    return [x_bc] + [t.to(pd) for t in ps]


def test_mamba2_proj_prologue_autograd_matches_finite_differences():
    """The projections composed with the element-wise prologue: every input's
    gradient (x_bc through four paths, the Dense kernels and bias) against
    central differences in float64."""
    B, L, H, P, N = 1, 5, 2, 2, 3
    ins = _m2x_inputs(B, L, H, P, N, 21)
    g = torch.Generator().manual_seed(22)
    cots = [torch.randn(B, L, H, P, generator=g, dtype=F64), torch.randn(B, L, H, P, generator=g, dtype=F64),
            torch.randn(B, L, N, generator=g, dtype=F64), torch.randn(B, L, N, generator=g, dtype=F64),
            torch.randn(H, generator=g, dtype=F64)]
    grads = op.mamba2_proj_prologue_grads(ins, cots, H, exact=True)

    def loss(args):
        return sum((o * c).sum() for o, c in zip(op.mamba2_proj_prologue(*args, H, exact=True), cots))

    h = 1e-6
    for i, t in enumerate(ins):
        fd = torch.zeros_like(t)
        for idx in range(t.numel()):
            e = torch.zeros(t.numel(), dtype=F64)
            e[idx] = h
            e = e.view(t.shape)
            p = list(ins); p[i] = t + e
            m = list(ins); m[i] = t - e
            fd.view(-1)[idx] = (loss(p) - loss(m)) / (2 * h)
        assert rel_err(grads[i], fd) < 1e-6, i


def test_mamba2_projections_match_linear_in_bf16():
    """bf16 dtype flow of the Dense layers: one rounding of the float32-accumulated
    product (torch.nn.functional.linear in float64, rounded), the bias added in
    bf16; the weight gradient is one rounding of x^T g, the bias gradient one
    rounding of the column sums, both returned as float32."""
    B, L, H, P, N = 2, 16, 2, 8, 8
    ins = _m2x_inputs(B, L, H, P, N, 23, dtype=torch.bfloat16)
    x, w_dt, b_dt, w_b = ins[0], ins[3], ins[4], ins[5]
    dt_pre, b_pre, _ = op.mamba2_projections(x, w_dt, b_dt, w_b, ins[6])
    lin = lambda w: torch.nn.functional.linear(x.double(), w.to(torch.bfloat16).double().t())
    assert torch.equal(b_pre, lin(w_b).to(torch.bfloat16))
    assert torch.equal(dt_pre, (lin(w_dt).to(torch.bfloat16) + b_dt.to(torch.bfloat16)))
    # gradients of the dt projection alone
    xl = x.clone().requires_grad_(True)
    wl = w_dt.clone().requires_grad_(True)
    bl = b_dt.clone().requires_grad_(True)
    gy = torch.randn(B, L, H * P, generator=torch.Generator().manual_seed(24)).to(torch.bfloat16)
    torch.autograd.backward(op.dense(xl, wl, bl), gy)
    assert wl.grad.dtype == torch.float32 and bl.grad.dtype == torch.float32
    x2 = x.double().reshape(-1, H * P)
    g2 = gy.double().reshape(-1, H * P)
    assert torch.equal(wl.grad, (x2.t() @ g2).to(torch.bfloat16).float())
    assert rel_err(bl.grad.double(), g2.sum(0)) < 1e-2      # bf16 sum of the cotangent rows
    assert torch.equal(xl.grad, (g2 @ w_dt.to(torch.bfloat16).double().t()).to(torch.bfloat16).reshape(x.shape))
