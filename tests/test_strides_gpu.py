"""Row-strided inputs through the C ABI (the args' row_stride): inputs that
are slices of a wider [B, T, F] tensor, e.g. the parts of a fused projection,
are read in place.  Every result must be bit-identical to the same call on
dense copies of those inputs."""
import pytest
import torch

from _util import banner
from atomic_ops import _lib, inputs
from atomic_ops import gdn2 as G
from atomic_ops import kernel_trainable_B6 as KT

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16


def _slices(ts, pad):
    """The tensors [B, T, H, D] as slices of one [B, T, sum(H D) + pad] tensor."""
    B, T = ts[0].shape[:2]
    widths = [t.shape[2] * t.shape[3] for t in ts]
    big = torch.zeros(B, T, sum(widths) + pad, dtype=ts[0].dtype, device="cuda")
    out, c = [], 0
    for t, wd in zip(ts, widths):
        big[..., c:c + wd] = t.reshape(B, T, wd).cuda()
        out.append(big[..., c:c + wd].view(t.shape))
        c += wd
    return out


def _gdn2_views(B, T, H, K, dtype, seed):
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype)
    q, k, v, w, b = _slices([d[n] for n in ("q", "k", "v", "w", "b")], 24)
    (g,) = _slices([d["g"]], 8)
    views = [q, k, v, w, b, g]
    for t in views:
        assert not t.is_contiguous() and G.rows(t)[1] == t.stride(1), "must be passed with its row stride"
    return views


@pytest.mark.parametrize("dtype,K", [(BF16, 128), (F32, 64)])
def test_gdn2_strided_inputs_equal_dense(dtype, K):
    B, T, H = 2, 256, 3
    banner(f"gdn2 row-strided inputs {dtype} K{K}")
    views = _gdn2_views(B, T, H, K, dtype, 7 + K)
    dense = [t.contiguous() for t in views]
    h0 = 0.2 * torch.randn(B, H, K, K, device="cuda")
    o_s, h_s, ws_s = G.forward(*views, 0.9, h0, save=True)
    o_d, h_d, ws_d = G.forward(*dense, 0.9, h0, save=True)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_d) and torch.equal(h_s, h_d)
    # upstream gradient as a slice too
    (dO,) = _slices([torch.randn(B, T, H, K).to(dtype)], 8)
    g_s = G.backward(*views, 0.9, dO, h0=h0, workspace=ws_s, reuse=True)
    g_d = G.backward(*dense, 0.9, dO.contiguous(), h0=h0, workspace=ws_d, reuse=True)
    g_r = G.backward(*views, 0.9, dO, h0=h0)   # recompute from the strided inputs
    torch.cuda.synchronize()
    for name, a, b_, c in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), g_s, g_d, g_r):
        assert a.is_contiguous() and torch.equal(a, b_) and torch.equal(c, b_), name


def test_gdn2_strided_noalloc_and_wrapper():
    B, T, H, K = 1, 512, 2, 128
    banner("gdn2 row-strided inputs: no-allocation forward, trainable wrapper")
    views = _gdn2_views(B, T, H, K, BF16, 21)
    dense = [t.contiguous() for t in views]
    o_s, h_s = G.forward_noalloc(*views, 1.0)
    o_d, h_d = G.forward_noalloc(*dense, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_d) and torch.equal(h_s, h_d)
    # the wrapper on views of two parents that require grad: the gradients
    # reach the parents' slices
    big = views[0]._base.detach().clone().requires_grad_(True)
    gbig = views[5]._base.detach().clone().requires_grad_(True)
    HK = H * K
    src = [big[..., i * HK:(i + 1) * HK].view(B, T, H, K) for i in range(5)] + [gbig[..., :HK].view(B, T, H, K)]
    leaves = [t.detach().clone().requires_grad_(True) for t in dense]
    o1, _ = KT.gdn2_pallas_forward_trainable(*src, 1.0)
    o2, _ = KT.gdn2_pallas_forward_trainable(*leaves, 1.0)
    cot = torch.randn_like(o1)
    torch.autograd.backward(o1, cot)
    torch.autograd.backward(o2, cot)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for i in range(5):
        assert torch.equal(big.grad[..., i * HK:(i + 1) * HK].reshape(B, T, H, K), leaves[i].grad), i
    assert torch.equal(gbig.grad[..., :HK].reshape(B, T, H, K), leaves[5].grad)


@pytest.mark.parametrize("dtype,C", [(BF16, 128), (F32, 64), (F32, 256)])
def test_mamba2_strided_inputs_equal_dense(dtype, C):
    """dt, x as slices of one [B, T, 2 H P + 8] tensor and B, C of one
    [B, T, 2 N + 8] tensor (the in_proj / projection outputs of a fused
    layer), dy a slice too: outputs and gradients bit-identical to dense
    (float32 operands: the float32 staged chain)."""
    from atomic_ops import mamba2 as M
    from atomic_ops import kernel_mamba2_trainable_B6 as KM
    B, T, H, P, N = 2, 512, 4, 64, 128
    banner(f"mamba2 row-strided inputs {dtype} chunk {C}")
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=31, dtype=dtype, dO=True)
    dt, x = _slices([d["dt"], d["x"]], 8)
    Bm, Cm = (t.view(B, T, N) for t in _slices([d["Bm"].view(B, T, 1, N), d["Cm"].view(B, T, 1, N)], 8))
    (dy,) = _slices([d["dy"]], 8)
    A = d["A"].cuda()
    views = [dt, x, Bm, Cm]
    for t in views + [dy]:
        assert not t.is_contiguous() and _lib.row_view(t)[1] == t.stride(1)
    dense = [t.contiguous() for t in views]
    s0 = 0.2 * torch.randn(B, H, P, N, device="cuda")
    y_s, f_s, ws_s = M.forward(*views, A, C, s0, save=True)
    y_d, f_d, ws_d = M.forward(*dense, A, C, s0, save=True)
    torch.cuda.synchronize()
    assert torch.equal(y_s, y_d) and torch.equal(f_s, f_d)
    g_s = M.backward(*views, A, C, dy, state0=s0, workspace=ws_s, reuse=True)
    g_d = M.backward(*dense, A, C, dy.contiguous(), state0=s0, workspace=ws_d, reuse=True)
    g_r = M.backward(*views, A, C, dy, state0=s0)
    torch.cuda.synchronize()
    for name, a, b_, c in zip(("ddt", "dx", "dB", "dC", "dA", "dstate0"), g_s, g_d, g_r):
        assert torch.equal(a, b_) and torch.equal(c, b_), name
    # the trainable wrapper on views of a parent that requires grad
    big = dt._base.detach().clone().requires_grad_(True)
    HP = H * P
    src = [big[..., :HP].view(B, T, H, P), big[..., HP:2 * HP].view(B, T, H, P), Bm, Cm]
    y1, _ = KM.mamba2_pallas_forward_trainable_B6(*src, A, C)
    leaves = [t.detach().clone().requires_grad_(True) for t in dense[:2]]
    y2, _ = KM.mamba2_pallas_forward_trainable_B6(leaves[0], leaves[1], dense[2], dense[3], A, C)
    torch.autograd.backward(y1, dy.float())
    torch.autograd.backward(y2, dy.float())
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(big.grad[..., :HP].reshape(B, T, H, P), leaves[0].grad)
    assert torch.equal(big.grad[..., HP:2 * HP].reshape(B, T, H, P), leaves[1].grad)
