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


def test_backward_exact_pairwise_path():
    """A chunk whose decay exceeds the factorisation bound takes the exact
    pairwise intra backward (with the reference's clip masks)."""
    banner("gdn2 bwd exact path")

    def mutate(inp):
        inp["g"][:, 64:128] *= 40.0
    args, ref = _case(1, 192, 2, 64, F32, seed=21, mutate=mutate)
    out = _gpu(args, 1.0, reuse=False)
    _check(out, ref, F32, (F32,) * 5 + (F32, F32))
