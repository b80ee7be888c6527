"""Writes the golden fixtures in this folder from the float64 oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its test files are
cited but absent), so these fixtures are held by this repository's oracle,
which tests/test_oracle_*.py pin by token-serial agreement, chunk-size
invariance, state passing, closed forms, finite differences and planted
mistakes.  Each fixture stores seeded inputs (bf16 as their uint16 bit
patterns) and the oracle's outputs and gradients rounded to float32.

  gdn2_small.npz    GDN2 fp32, config 0 distributions, B1 T128 H1 K=V=64 C64,
                    scale 1, random h0 and dh_final
  gdn2_bf16.npz     GDN2 bf16 inputs, B1 T128 H1 K=V=128 C64, h0 = 0
  mamba2_small.npz  Mamba2 bf16 inputs, config 1 distributions, B1 T256 H1 P64
                    N64 C128, random state0 and dstate_final
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "atomic_ai_hybrid-v0.1_amd")]

from atomic_ops import inputs  # noqa: E402
from oracle import gdn2 as og, mamba2 as om  # noqa: E402


def _np(t):
    """bf16 tensors as their uint16 bit patterns (exact), others as float32."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.to(torch.float32).numpy()


def load(name):
    """Fixture ``name`` as a dict of torch tensors (bf16 restored)."""
    out = {}
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        for n in z.files:
            a = z[n]
            if a.dtype == np.uint16:
                out[n] = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
            elif a.dtype.kind == "f" and a.ndim > 0:
                out[n] = torch.from_numpy(a.copy())
            else:
                out[n] = a.item() if a.ndim == 0 and a.dtype.kind != "U" else str(a)
    return out


def gdn2_case(name, B, T, H, K, dtype, seed, with_state):
    d = inputs.gdn2_inputs(B, T, H, K, K, seed=seed, dtype=dtype, dO=True)
    gen = torch.Generator().manual_seed(seed + 100)
    h0 = 0.3 * torch.randn(B, H, K, K, generator=gen) if with_state else None
    dht = torch.randn(B, H, K, K, generator=gen) if with_state else None
    q, k, v, w, b, g, do = (d[n] for n in ("q", "k", "v", "w", "b", "g", "do"))
    o, h = og.gdn2_chunked_wy_reference(q, k, v, g, b, w, 1.0, 64, h0=h0)
    grads = og.gdn2_backward_autodiff(q, k, v, w, b, g, 1.0, 64, do, dh_final=dht, h0=h0)
    arrs = dict(q=q, k=k, v=v, w=w, b=b, g=g, do=do, o=o, h_final=h)
    arrs.update(zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads))
    if with_state:
        arrs.update(h0=h0, dh_final=dht)
    np.savez_compressed(os.path.join(HERE, name), dtype=str(dtype).split(".")[-1], chunk=64,
                        scale=1.0, **{n: _np(t) for n, t in arrs.items()})


def mamba2_case(name, B, T, H, P, N, C, seed):
    d = inputs.mamba2_inputs(B, T, H, P, N, seed=seed, dO=True)
    gen = torch.Generator().manual_seed(seed + 100)
    s0 = 0.3 * torch.randn(B, H, P, N, generator=gen)
    dsf = torch.randn(B, H, P, N, generator=gen)
    dt, x, Bm, Cm, A, dy = (d[n] for n in ("dt", "x", "Bm", "Cm", "A", "dy"))
    y, s = om.mamba2_ssd_reference(dt, A, Bm, Cm, x, C, state0=s0)
    ddt, dB, dC, dx, dA, ds0 = om.chunk_ssd_bwd_scan(dt, A, Bm, Cm, x, C, dy, dsf, state0=s0)
    arrs = dict(dt=dt, x=x, Bm=Bm, Cm=Cm, A=A, dy=dy, state0=s0, dstate_final=dsf, y=y,
                state_final=s, ddt=ddt, dB=dB, dC=dC, dx=dx, dA=dA, dstate0=ds0)
    np.savez_compressed(os.path.join(HERE, name), dtype="bfloat16", chunk=C,
                        **{n: _np(t) for n, t in arrs.items()})


def main():
    gdn2_case("gdn2_small.npz", 1, 128, 1, 64, torch.float32, seed=20, with_state=True)
    gdn2_case("gdn2_bf16.npz", 1, 128, 1, 128, torch.bfloat16, seed=21, with_state=False)
    mamba2_case("mamba2_small.npz", 1, 256, 1, 64, 64, 128, seed=22)


if __name__ == "__main__":
    main()
