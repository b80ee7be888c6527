"""Mamba2 SSD forward on the GPU (through the C ABI) against the CPU oracle."""
import pytest
import torch

from _util import banner, rel_err, tol_for
from atomic_ops import inputs
from atomic_ops import mamba2 as M
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _run(B, T, H, P, N, C, seed, state=False, mutate=None, **kw):
    inp = inputs.mamba2_inputs(B, T, H, P, N, seed=seed, **kw)
    if mutate:
        mutate(inp)
    dt, x, Bm, Cm, A = (inp[n] for n in ("dt", "x", "Bm", "Cm", "A"))
    s0 = 0.3 * torch.randn(B, H, P, N, generator=torch.Generator().manual_seed(seed + 1)) if state else None
    y_ref, s_ref = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0)
    y, s, _ = M.forward(dt.cuda(), x.cuda(), Bm.cuda(), Cm.cuda(), A.cuda(), C,
                        state0=s0.cuda() if state else None)
    torch.cuda.synchronize()
    return (y, s), (y_ref, s_ref)


@pytest.mark.parametrize("B,T,H,P,N,C,state", [
    (2, 512, 4, 64, 128, 128, False),     # config 1 head shape (T reduced)
    (1, 384, 3, 64, 128, 128, True),
    (1, 256, 2, 128, 128, 128, True),     # headline P=128
    (2, 256, 2, 64, 128, 64, False),      # chunk 64
    (1, 256, 2, 64, 64, 128, True),       # N = 64
    (1, 512, 2, 192, 128, 256, True),     # the model's call site: headdim 192, chunk_size 256
    (2, 256, 3, 192, 128, 128, False),    # headdim 192, chunk 128
])
def test_forward_matches_oracle(B, T, H, P, N, C, state):
    banner(f"mamba2 fwd B{B} T{T} H{H} P{P} N{N} C{C} state={state}")
    (y, s), (y_ref, s_ref) = _run(B, T, H, P, N, C, seed=T + P + C, state=state)
    ey, es = rel_err(y, y_ref), rel_err(s, s_ref)
    print(f"  rel_err y={ey:.3e} state={es:.3e}")
    assert torch.isfinite(y).all() and torch.isfinite(s).all()
    assert ey < tol_for(BF16) and es < tol_for(BF16)


def test_positive_step_exponent_takes_exact_path():
    """dt A > 0 somewhere (A > 0 for one head) breaks the monotone decay; that
    chunk is evaluated pairwise with the reference's clips."""
    banner("mamba2 fwd positive exponent")

    def mutate(inp):
        inp["A"][1] = 0.05
    (y, s), (y_ref, s_ref) = _run(1, 256, 3, 64, 128, 128, seed=5, mutate=mutate)
    ey, es = rel_err(y, y_ref), rel_err(s, s_ref)
    print(f"  rel_err y={ey:.3e} state={es:.3e}")
    assert ey < tol_for(BF16) and es < tol_for(BF16)


def test_steep_decay_takes_exact_path():
    """A = -200 for one head: step exponents past the -20 clip and 16-row
    block ranges far beyond the factorisation bound, so that head's slices
    are evaluated pairwise with the reference's clips."""
    banner("mamba2 fwd steep decay")

    def mutate(inp):
        inp["A"][1] = -200.0
    (y, s), (y_ref, s_ref) = _run(1, 256, 3, 64, 128, 128, seed=7, mutate=mutate)
    ey, es = rel_err(y, y_ref), rel_err(s, s_ref)
    print(f"  rel_err y={ey:.3e} state={es:.3e}")
    assert ey < tol_for(BF16) and es < tol_for(BF16)


def test_decay_weight_cap():
    """A positive step exponent (A = +1) drives exp(clip(cum_i - cum_j, +-20))
    past the reference's 1e6 cap on L (mamba2_ssd_reference.py:120) for the
    far pairs of a chunk.  One chunk, so y is y_diag alone, which the exact
    path evaluates pairwise in fp32.  The capped terms reach ~1e4, where the
    bf16 rounding of the shared CB scores would dominate a sum with
    cancellation, so x, B and C are made non-negative: every term is then
    positive and the comparison isolates the cap.  x is scaled by 1e-3 so
    that y stays below the 1e4 output clip; there the uncapped weights would
    change y by about 2x its maximum."""
    banner("mamba2 fwd L cap")

    def mutate(inp):
        inp["A"][0] = 1.0
        for n in ("x", "Bm", "Cm"):
            inp[n] = inp[n].abs()
        inp["x"] = (inp["x"].float() * 1e-3).to(inp["x"].dtype)
    (y, s), (y_ref, s_ref) = _run(1, 128, 2, 64, 128, 128, seed=6, mutate=mutate)
    dt = inputs.mamba2_inputs(1, 128, 2, 64, 128, seed=6)["dt"].double()
    cum = torch.cumsum(dt[0, :, 0], 0)
    assert (cum[-1] - cum[0]).max() > 13.9, "the cap must be reached"
    ey = rel_err(y, y_ref)
    print(f"  rel_err y={ey:.3e}")
    assert ey < tol_for(BF16)
