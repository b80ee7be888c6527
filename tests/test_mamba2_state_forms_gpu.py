"""The two forms of the Mamba2 state loops give the same results.

When the (batch, head, 32-channel) workgroups fill the 256 CUs, the state
loops walk the chunks forming each chunk's S^T B (forward) or Ydh^T C
(backward) on MFMA (mamba2_seq.hpp); smaller grids run the two-pass form
(the chunk kernel writes each chunk's fp32 product, an element-wise pass
carries the state).  Heads are independent, so the first four heads of a
wide run (which takes the loops) and the same four heads run alone (which
take the two passes) must agree: the states are the same MFMA over the same
bf16 operands followed by the same recurrence, so y, the final state, dx and
dstate0 are equal bit for bit; ddt and dA take the decay_chunk_end row term,
whose sum over the state columns runs in another order (float32 rounding).
Reference semantics: mamba2_ssd_reference.py:133-146 and
mamba2_bwd_reference.py:115-135,195.
"""
import pytest
import torch

from _util import banner, rel_err
from atomic_ops import inputs
from atomic_ops import mamba2 as M

pytestmark = pytest.mark.gpu

SUB = 4  # heads of the two-pass run: B * SUB * P / 32 workgroups, far below 256


@pytest.mark.parametrize("B,T,H,P,N,C", [(1, 512, 128, 64, 128, 128), (2, 256, 32, 128, 64, 64)])
def test_state_loop_forms_agree(B, T, H, P, N, C):
    assert B * H * (P // 32) >= 256 and B * SUB * (P // 32) < 256
    banner(f"mamba2 state loop forms B{B} T{T} H{H} P{P} N{N} C{C}")
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=71, device=torch.device("cuda"), dO=True)
    dt, x, Bm, Cm, A, dy = (d[n] for n in ("dt", "x", "Bm", "Cm", "A", "dy"))
    gen = torch.Generator(device="cuda").manual_seed(72)
    s0 = 0.3 * torch.randn(B, H, P, N, device="cuda", generator=gen)
    dsf = 0.3 * torch.randn(B, H, P, N, device="cuda", generator=gen)

    def heads(t):
        return t[:, :, :SUB].contiguous()

    y_w, sf_w, _ = M.forward(dt, x, Bm, Cm, A, C, state0=s0)
    g_w = M.backward(dt, x, Bm, Cm, A, C, dy, dstate_final=dsf, state0=s0)
    y_s, sf_s, _ = M.forward(heads(dt), heads(x), Bm, Cm, A[:SUB].contiguous(), C,
                             state0=s0[:, :SUB].contiguous())
    g_s = M.backward(heads(dt), heads(x), Bm, Cm, A[:SUB].contiguous(), C, heads(dy),
                     dstate_final=dsf[:, :SUB].contiguous(), state0=s0[:, :SUB].contiguous())
    torch.cuda.synchronize()
    ddt_w, dx_w, _, _, dA_w, ds0_w = g_w
    ddt_s, dx_s, _, _, dA_s, ds0_s = g_s
    e_ddt = rel_err(heads(ddt_w), ddt_s)
    e_da = rel_err(dA_w[:SUB], dA_s)
    print(f"  ddt rel_err {e_ddt:.2e}  dA rel_err {e_da:.2e}", flush=True)
    assert torch.equal(heads(y_w), y_s)
    assert torch.equal(sf_w[:, :SUB], sf_s)
    assert torch.equal(heads(dx_w), dx_s)
    assert torch.equal(ds0_w[:, :SUB], ds0_s)
    assert e_ddt < 1e-5 and e_da < 1e-5
