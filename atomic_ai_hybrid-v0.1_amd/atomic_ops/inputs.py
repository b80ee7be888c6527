"""Seeded synthetic inputs for the GDN2 and Mamba2 chunk paths.

The distributions are the ones the benchmark configurations name:

GDN2 (q, k, b, g: [B,T,H,K]; v, w: [B,T,H,V])
  q, k ~ N(0,1), L2-normalised over K      (as model.py:597-601)
  v    ~ N(0,1)
  b    = sigmoid(N(0,1))   per channel     (erase gate, model.py:603)
  w    = sigmoid(N(0,1))   per channel     (write gate, model.py:604)
  g    = log(sigmoid(N(3,1)))  float32, every entry negative
Mamba2 (dt, x: [B,T,H,P]; Bm, Cm: [B,T,N]; A: [H])
  x  ~ N(0,1)
  dt = softplus(N(-2, 0.5))  per head and channel (model.py:427)
  A  = -exp(U(log 1, log 16))  float32
  Bm, Cm ~ N(0,1) / sqrt(N)

Low-precision storage: q,k,v,b,w (GDN2) and dt,x,B,C (Mamba2) are rounded
to ``dtype``; g and A stay float32 (model.py:609, model.py:423).
"""
from __future__ import annotations

import math

import torch


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def gdn2_inputs(B, T, H, K, V, *, seed=0, dtype=torch.bfloat16, device="cpu",
                dO=False, g_mean=3.0):
    """Returns a dict with q,k,v,w,b (``dtype``), g (float32) and, when
    ``dO`` is set, an upstream gradient ``do`` ~ N(0,1) in ``dtype``."""
    gen = _gen(seed, device)
    f32 = torch.float32
    q = torch.randn(B, T, H, K, generator=gen, device=device, dtype=f32)
    k = torch.randn(B, T, H, K, generator=gen, device=device, dtype=f32)
    q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-12)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-12)
    v = torch.randn(B, T, H, V, generator=gen, device=device, dtype=f32)
    b = torch.sigmoid(torch.randn(B, T, H, K, generator=gen, device=device, dtype=f32))
    w = torch.sigmoid(torch.randn(B, T, H, V, generator=gen, device=device, dtype=f32))
    g = torch.nn.functional.logsigmoid(
        g_mean + torch.randn(B, T, H, K, generator=gen, device=device, dtype=f32))
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), w=w.to(dtype), b=b.to(dtype),
               g=g.contiguous())
    if dO:
        out["do"] = torch.randn(B, T, H, V, generator=gen, device=device, dtype=f32).to(dtype)
    return out


def mamba2_inputs(B, T, H, P, N, *, seed=0, dtype=torch.bfloat16, device="cpu", dO=False,
                  dt_mean=-2.0, dt_std=0.5, a_max=16.0):
    """Returns a dict with dt, x, Bm, Cm (``dtype``), A (float32) and, when
    ``dO`` is set, an upstream gradient ``dy`` ~ N(0,1) in ``dtype``."""
    gen = _gen(seed, device)
    f32 = torch.float32
    x = torch.randn(B, T, H, P, generator=gen, device=device, dtype=f32)
    dt = torch.nn.functional.softplus(
        dt_mean + dt_std * torch.randn(B, T, H, P, generator=gen, device=device, dtype=f32))
    u = torch.rand(H, generator=gen, device=device, dtype=f32)
    A = -torch.exp(u * math.log(a_max))
    Bm = torch.randn(B, T, N, generator=gen, device=device, dtype=f32) / math.sqrt(N)
    Cm = torch.randn(B, T, N, generator=gen, device=device, dtype=f32) / math.sqrt(N)
    out = dict(dt=dt.to(dtype), x=x.to(dtype), Bm=Bm.to(dtype), Cm=Cm.to(dtype),
               A=A.contiguous())
    if dO:
        out["dy"] = torch.randn(B, T, H, P, generator=gen, device=device, dtype=f32).to(dtype)
    return out
