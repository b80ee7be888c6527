"""Mamba2 stage-level forward on the GPU, through the C ABI: M2
(``build_chunk_cumdecay_pallas``, kernel_mamba2_a_decay.py:71), M3
(``intra_chunk_ssd_pallas``, kernel_mamba2_b_intra.py:119), M4
(``mamba2_inter_chunk_combine``, kernel_mamba2_c_interchunk.py:38) and the
staged ``mamba2_pallas_forward`` (:90).  Each stage on the oracle's inputs to
that stage, against the oracle's restatement of it (cumdecay fp32 to 1e-4,
the rest to the bf16 bound 2e-2); the staged forward bit-identical to the
whole-path forward while no clip binds, and against the stage oracle where a
positive step exponent makes the stage kernels' clips differ from the whole
path's."""
import pytest
import torch

from _util import TOL_BF16, TOL_F32, banner, rel_err
from atomic_ops import _lib, inputs
from atomic_ops import kernel_mamba2_a_decay as MA
from atomic_ops import kernel_mamba2_b_intra as MB
from atomic_ops import kernel_mamba2_c_interchunk as MC
from atomic_ops import mamba2 as M
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu


def _inp(B, T, H, P, N, seed, mutate=None):
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=seed)
    if mutate:
        mutate(d)
    return [d[n] for n in ("dt", "x", "Bm", "Cm", "A")]


def _check(name, got, ref, tol):
    e = rel_err(got, ref)
    print(f"  {name}: rel_err {e:.2e}")
    assert got.shape == ref.shape and got.dtype == torch.float32 and e < tol, name


@pytest.mark.parametrize("B,T,H,P,N,C", [
    (2, 256, 3, 64, 128, 128),
    (1, 256, 2, 128, 64, 64),
    (1, 384, 2, 128, 128, 128),
    (1, 256, 2, 192, 128, 128),    # the model's headdim
])
def test_each_stage_matches_the_oracle(B, T, H, P, N, C):
    banner(f"mamba2 stages B{B} T{T} H{H} P{P} N{N} C{C}")
    dt, x, Bm, Cm, A = _inp(B, T, H, P, N, seed=T + P + N + C)
    s0 = 0.3 * torch.randn(B, H, P, N, generator=torch.Generator().manual_seed(7))
    s0[0, 0, 0, 0], s0[0, -1, 1, 1] = float("nan"), 3e4         # sanitised by M4
    cum_ref = om.build_chunk_cumdecay(dt, A, C)
    yd_ref, se_ref = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_ref, C)
    y_ref, sf_ref = om.mamba2_inter_chunk_combine(yd_ref, se_ref, cum_ref, Cm, C, state0=s0)
    g = [t.cuda() for t in (dt, x, Bm, Cm, A)]
    cum = MA.build_chunk_cumdecay_pallas(g[0], g[4], C)
    yd, se = MB.intra_chunk_ssd_pallas(g[0], g[1], g[2], g[3], cum_ref.float().cuda(), C)
    y, sf = MC.mamba2_inter_chunk_combine(yd_ref.float().cuda(), se_ref.float().cuda(), cum_ref.float().cuda(),
                                          g[3], C, state0=s0.cuda())
    torch.cuda.synchronize()
    _check("cumdecay", cum, cum_ref, TOL_F32)
    _check("y_diag", yd, yd_ref, TOL_BF16)
    _check("state_end", se, se_ref, TOL_BF16)
    _check("y", y, y_ref, TOL_BF16)
    _check("state_final", sf, sf_ref, TOL_BF16)


@pytest.mark.parametrize("B,T,H,P,N,C", [(2, 512, 4, 128, 128, 128), (1, 256, 3, 64, 64, 64)])
def test_staged_forward_equals_the_whole_forward(B, T, H, P, N, C):
    """Every step exponent negative and a moderate state0: the stage kernels'
    clips and the whole path's give the same numbers and the stages run the
    same kernels.  state_final comes out bit-identical.  y differs by the
    rounding of the cum: the whole path's output kernel sums it over
    32-channel slices (8 row segments), the cumdecay kernel over 64-channel
    slices (4 row segments); with |cum| ~ 250 at the chunk end (fp32 ulp
    3e-5) a few ulps move exp(cum_i - cum_j) by ~1e-4 relative."""
    banner(f"mamba2 staged vs whole B{B} T{T} H{H} P{P} N{N} C{C}")
    g = [t.cuda() for t in _inp(B, T, H, P, N, seed=11)]
    s0 = 0.3 * torch.randn(B, H, P, N, device="cuda")
    y_w, s_w, _ = M.forward(*g, C, state0=s0)
    y_s, s_s = MC.mamba2_pallas_forward(g[0], g[1], g[2], g[3], g[4], C, state0=s0)
    torch.cuda.synchronize()
    e = rel_err(y_s, y_w)
    print(f"  y: rel_err {e:.2e}")
    assert torch.equal(s_s, s_w) and e < 2e-3


def test_positive_exponent_follows_the_stage_kernels():
    """A = +1 for one head: pair weights reach exp(20) and the chunk's write
    passes 1e4.  The staged forward follows the stage kernels (no 1e6 caps, a
    sanitised write), which the whole-path oracle does not; x, B, C are
    non-negative so that bf16 rounding of the shared CB scores does not meet
    cancellation (the terms reach ~1e4), and x is scaled down so y stays
    below the 1e4 output clip."""
    banner("mamba2 staged forward, positive exponent")

    def mutate(d):
        d["A"][0] = 1.0
        for n in ("x", "Bm", "Cm"):
            d[n] = d[n].abs()
        d["x"] = (d["x"].float() * 1e-3).to(d["x"].dtype)
    dt, x, Bm, Cm, A = _inp(1, 256, 2, 64, 128, seed=6, mutate=mutate)
    cum_ref = om.build_chunk_cumdecay(dt, A, 128)
    yd_ref, se_ref = om.intra_chunk_ssd(dt, x, Bm, Cm, cum_ref, 128)
    y_ref, sf_ref = om.mamba2_inter_chunk_combine(yd_ref, se_ref, cum_ref, Cm, 128)
    y_whole, _ = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, 128)
    assert rel_err(y_whole, y_ref) > 0.1, "the caps must bind"
    y, sf = MC.mamba2_pallas_forward(*(t.cuda() for t in (dt, x, Bm, Cm, A)), 128)
    torch.cuda.synchronize()
    _check("y", y, y_ref, TOL_BF16)
    _check("state_final", sf, sf_ref, TOL_BF16)
