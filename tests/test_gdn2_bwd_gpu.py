"""GDN2 backward on the GPU (through the C ABI) against the oracle: the
gradient of the chunked WY reference (torch autograd, float64), i.e. the
meaning of kernel_trainable.py:38-55, with the final clip of
kernel_trainable_B6.py:173-179."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import gdn2 as G
from atomic_ops import inputs
from oracle import gdn2 as og

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
NAMES = ("dq", "dk", "dv", "dw", "db", "dg", "dh0")


def _case(B, T, H, K, dtype, seed, scale=1.0, with_state=False, do_dtype=None, mutate=None):
    inp = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype, dO=True)
    if mutate:
        mutate(inp)
    q, k, v, w, b, g, dO = (inp[n] for n in "q k v w b g do".split())
    if do_dtype is not None:
        dO = dO.to(do_dtype)
    gen = torch.Generator().manual_seed(seed + 5)
    h0 = 0.3 * torch.randn(B, H, K, K, generator=gen) if with_state else None
    dh = torch.randn(B, H, K, K, generator=gen) if with_state else None
    ref = og.gdn2_backward_autodiff(q, k, v, w, b, g, scale, 64, dO, dh, h0=h0)
    return (q, k, v, w, b, g, dO, h0, dh), ref


def _gpu(args, scale, reuse):
    q, k, v, w, b, g, dO, h0, dh = (t.cuda() if t is not None else None for t in args)
    ws = None
    if reuse:
        _, _, ws = G.forward(q, k, v, w, b, g, scale, h0=h0, save=True)
    out = G.backward(q, k, v, w, b, g, scale, dO, dh_final=dh, h0=h0, workspace=ws, reuse=reuse)
    torch.cuda.synchronize()
    return out


def _check(out, ref, dtype, primal_dtypes):
    tol = tol_for(dtype)
    errs = {}
    for name, got, want, pdt in zip(NAMES, out, ref, primal_dtypes):
        assert got.dtype == pdt, (name, got.dtype, pdt)
        assert torch.isfinite(got).all(), name
        errs[name] = rel_err(got, want)
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for name, e in errs.items():
        assert e < tol, (name, e)


@pytest.mark.parametrize("B,T,H,K,dtype,scale,with_state,reuse", [
    (1, 256, 2, 64, F32, 1.0, False, False),          # config 0 head shape
    (1, 192, 2, 64, F32, 0.125, True, True),
    (1, 192, 2, 128, BF16, 1.0, False, True),         # config 2/3 head shape
    (2, 128, 2, 128, BF16, 128 ** -0.5, True, False),
    (1, 128, 2, 64, BF16, 1.0, True, True),
    (1, 64, 2, 128, BF16, 1.0, True, True),           # one chunk: only the state loop's tail step
    (1, 128, 48, 128, BF16, 1.0, True, True),         # 48 heads: 32-column V tiles in the forward
    (1, 192, 2, 128, F32, 128 ** -0.5, True, True),   # fp32 operands at K = 128 (fp32 tolerance)
    (2, 128, 3, 128, F32, 1.0, False, False),
])
def test_backward_matches_autodiff(B, T, H, K, dtype, scale, with_state, reuse):
    banner(f"gdn2 bwd B{B} T{T} H{H} K{K} {dtype} scale={scale} state={with_state} reuse={reuse}")
    args, ref = _case(B, T, H, K, dtype, seed=3 * K + T, scale=scale, with_state=with_state)
    out = _gpu(args, scale, reuse)
    _check(out, ref, dtype, (dtype,) * 5 + (F32, F32))


def test_backward_fp32_upstream_gradient():
    """dO arriving as float32 (the reference's o is float32) with bf16 primals."""
    banner("gdn2 bwd bf16 primals, fp32 dO")
    args, ref = _case(1, 128, 2, 128, BF16, seed=17, do_dtype=F32)
    out = _gpu(args, 1.0, reuse=False)
    _check(out, ref, BF16, (BF16,) * 5 + (F32, F32))


@pytest.mark.parametrize("case,dtype,K", [
    ("deep_decay", F32, 64), ("deep_decay", BF16, 128), ("deep_decay_upper_columns", BF16, 128),
    ("positive_gate", BF16, 128), ("deep_decay_upper_columns", F32, 128),
])
def test_backward_exact_pairwise_path(case, dtype, K):
    """A chunk whose decay exceeds the factorisation bound takes the exact
    pairwise intra backward (with the reference's clip masks).  The intra
    backward decides per 64-column slice: in the upper-columns case chunk 1
    mixes a factorised slice (columns 0..63) with an exact one (64..127)."""
    banner(f"gdn2 bwd exact path {case} {dtype} K{K}")

    def mutate(inp):
        g = inp["g"]
        if case == "deep_decay":
            g[:, 64:128] *= 40.0
        elif case == "positive_gate":
            g[:, 70:74] = 0.4
        else:
            g[:, 64:128, :, 64:] *= 40.0
    args, ref = _case(1, 192, 2, K, dtype, seed=21, mutate=mutate)
    out = _gpu(args, 1.0, reuse=False)
    _check(out, ref, dtype, (dtype,) * 5 + (F32, F32))


@pytest.mark.parametrize("h0_given,use_h_final", [(False, False), (True, True)])
def test_trainable_wrapper_autograd(h0_given, use_h_final):
    """gdn2_pallas_forward_trainable (kernel_trainable_B6.py:187-194) through
    torch.autograd: primal dtypes kept on every gradient, equal to the direct
    forward / backward calls, within tolerance of the oracle; a second
    backward through the retained graph (which recomputes the forward's
    intermediates) gives the same gradients."""
    from atomic_ops.kernel_trainable_B6 import gdn2_pallas_forward_trainable
    B, T, H, K = 1, 192, 2, 128
    banner(f"gdn2 trainable wrapper h0={h0_given} h_final used={use_h_final}")
    inp = inputs.gdn2_inputs(B, T, H, K, K, seed=31, dtype=BF16, dO=True)
    gen = torch.Generator().manual_seed(32)
    h0 = 0.3 * torch.randn(B, H, K, K, generator=gen) if h0_given else None
    dh = torch.randn(B, H, K, K, generator=gen) if use_h_final else None
    names = ("q", "k", "v", "w", "b", "g")
    dev = {n: inp[n].cuda() for n in names + ("do",)}
    leaves = [dev[n].clone().requires_grad_(True) for n in names]
    h0l = h0.cuda().requires_grad_(True) if h0_given else None
    o, hf = gdn2_pallas_forward_trainable(*leaves, 1.0, h0l)
    assert o.dtype == torch.float32 and hf.dtype == torch.float32
    loss = (o * dev["do"].float()).sum()
    if use_h_final:
        loss = loss + (hf * dh.cuda()).sum()
    loss.backward(retain_graph=True)
    wrt = leaves + ([h0l] if h0_given else [])
    first = [t.grad.clone() for t in wrt]
    for t in wrt:
        assert t.grad.dtype == t.dtype
    direct = G.backward(*(dev[n] for n in names), 1.0, dev["do"].float(),
                        dh_final=dh.cuda() if use_h_final else None,
                        h0=h0.cuda() if h0_given else None)
    for got, want in zip(first, direct[:6] + (direct[6],) if h0_given else direct[:6]):
        assert torch.equal(got, want) or rel_err(got, want) < 1e-6
    ref = og.gdn2_backward_autodiff(*(inp[n] for n in names), 1.0, 64, inp["do"], dh, h0=h0)
    errs = {n: rel_err(g_, r) for n, g_, r in zip(NAMES, first, ref)}
    print("  rel_err " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for n, e in errs.items():
        assert e < tol_for(BF16), (n, e)
    for t in wrt:
        t.grad = None
    loss.backward()
    for t, want in zip(wrt, first):
        assert torch.equal(t.grad, want) or rel_err(t.grad, want) < 1e-6


@pytest.mark.parametrize("chunk,dtype,K,g_mean", [
    (128, F32, 64, 0.0), (256, F32, 64, 0.0), (256, BF16, 128, 3.0),
])
def test_longer_chunks_match_the_oracle_at_that_chunk(chunk, dtype, K, g_mean):
    """chunk_size 128 / 256 (the reference's Pallas path runs 256,
    kernel_a_scores.py:15-17) against the oracle at that chunk size, forward
    and backward; the kernels run 64-row chunks.  With g_mean 0 the decay is
    about -0.7 per step, so the reference's exp(-20) floor fires on the far
    pairs of the longer chunks."""
    banner(f"gdn2 chunk {chunk} {dtype} K{K} g_mean={g_mean}")
    B, T, H = 1, 512, 2
    inp = inputs.gdn2_inputs(B, T, H, K, K, seed=chunk + K, dtype=dtype, dO=True, g_mean=g_mean)
    q, k, v, w, b, g, dO = (inp[n] for n in "q k v w b g do".split())
    h0 = 0.3 * torch.randn(B, H, K, K, generator=torch.Generator().manual_seed(chunk))
    o_ref, h_ref = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, chunk, h0=h0)
    ref = og.gdn2_backward_autodiff(q, k, v, w, b, g, 1.0, chunk, dO, None, h0=h0)
    dev = [t.cuda() for t in (q, k, v, w, b, g)]
    o, hf, ws = G.forward(*dev, 1.0, h0=h0.cuda(), save=True, chunk=chunk)
    out = G.backward(*dev, 1.0, dO.cuda(), h0=h0.cuda(), workspace=ws, reuse=True, chunk=chunk)
    torch.cuda.synchronize()
    eo, eh = rel_err(o, o_ref), rel_err(hf, h_ref)
    print(f"  rel_err o={eo:.2e} h_final={eh:.2e}")
    assert eo < tol_for(dtype) and eh < tol_for(dtype)
    _check(out, ref, dtype, (dtype,) * 5 + (F32, F32))


def test_reuse_requires_the_matching_forward():
    """REUSE on a workspace that holds another forward is refused before any
    launch: other input tensors (same shapes), and the workspace overwritten by
    another call of the library since; the matching forward reuses as before,
    and a non-contiguous input turns reuse into a recompute (same gradients)."""
    from atomic_ops import _lib
    from atomic_ops import norm_gate as NG
    banner("gdn2 reuse tag")
    args, _ = _case(1, 128, 2, 64, BF16, 41)
    q, k, v, w, b, g, dO, _, _ = (t.cuda() if t is not None else None for t in args)
    _, _, ws = G.forward(q, k, v, w, b, g, 1.0, save=True)
    with pytest.raises(_lib.AtomicError, match="REUSE"):
        G.backward(q.clone(), k, v, w, b, g, 1.0, dO, workspace=ws, reuse=True)
    ref = G.backward(q, k, v, w, b, g, 1.0, dO, workspace=ws, reuse=True)
    again = G.backward(q, k, v, w, b, g, 1.0, dO, workspace=ws, reuse=True)   # the forward is still there
    for a, r in zip(again, ref):
        assert torch.equal(a, r)
    # another entry point writes the workspace: its record is gone
    rows, d = 64, 512
    x = torch.randn(rows, d, device="cuda")
    gate = torch.randn(rows, d, device="cuda").to(BF16)
    NG.backward(x, gate, torch.ones(d, device="cuda"), torch.randn(rows, d, device="cuda").to(BF16), NG.GDN2,
                workspace=ws)
    with pytest.raises(_lib.AtomicError, match="REUSE"):
        G.backward(q, k, v, w, b, g, 1.0, dO, workspace=ws, reuse=True)
    # a transposed-and-back (non-contiguous) input is copied, so the call recomputes
    _, _, ws = G.forward(q, k, v, w, b, g, 1.0, save=True)
    qn = q.transpose(1, 2).contiguous().transpose(1, 2)
    assert not qn.is_contiguous()
    got = G.backward(qn, k, v, w, b, g, 1.0, dO, workspace=ws, reuse=True)
    torch.cuda.synchronize()
    for a, r in zip(got, ref):
        assert torch.equal(a, r)


def test_nonfinite_do_gives_finite_gradients():
    """A NaN and an inf in dO: every gradient is finite and inside the final
    clip (kernel_trainable_B6.py:173-179).  The autodiff oracle multiplies
    its causal masks in, so a non-finite dO row also poisons the masked pairs
    (NaN x 0) before the sanitising clips; the kernels skip those pairs, so
    the values are not compared (the model's gradient sanitiser,
    model.py:192-217, keeps dO finite)."""
    banner("gdn2 bwd non-finite dO")

    def mutate(inp):
        inp["do"][0, 10, 1, 5] = float("nan")
        inp["do"][0, 70, 0, 3] = float("inf")
    args, _ = _case(1, 128, 2, 128, BF16, seed=41, with_state=True, mutate=mutate)
    out = _gpu(args, 1.0, reuse=True)
    for name, got in zip(NAMES, out):
        assert torch.isfinite(got).all(), name
        assert got.abs().max().item() <= 1e4, name
