"""Seeded input builders shared by the tests (CPU generator, then moved)."""
import torch


def randn(shape, seed, dtype=torch.bfloat16, device="cpu", scale=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32) * scale
    return x.to(dtype).to(device)


def max_abs(a, b):
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    both_nan = torch.isnan(a) & torch.isnan(b)
    d = (a - b).abs()
    d[both_nan] = 0
    return float(d.max()) if d.numel() else 0.0
