import torch

TOL_F32 = 1e-4   # north-star tolerance, fp32 configs
TOL_BF16 = 2e-2  # north-star tolerance, bf16 inputs with fp32 accumulation


def rel_err(a, b):
    """Norm-wise max relative error max|a - b| / max|b| (float64, on CPU)."""
    a = a.detach().to("cpu", torch.float64)
    b = b.detach().to("cpu", torch.float64)
    den = b.abs().max().item()
    return (a - b).abs().max().item() / max(den, 1e-300)


def tol_for(dtype):
    return TOL_F32 if dtype == torch.float32 else TOL_BF16


def banner(msg):
    print(f"[case] {msg}", flush=True)
