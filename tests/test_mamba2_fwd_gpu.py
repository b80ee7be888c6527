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
