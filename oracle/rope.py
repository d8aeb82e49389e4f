"""CPU restatement of the reference's RoPE tables, rotation and KV append.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import math

import torch


def inv_freq(dim: int, theta: float, rope_scaling: dict | None = None) -> torch.Tensor:
    """fp32 inverse frequencies (src/rope.py:8-30).

    base: 1 / theta^(2i/dim) in fp32 (:9).  With llama3 scaling (:14-30), by
    wavelength 2*pi/f: above old_ctx/low_freq_factor -> f/factor; below
    old_ctx/high_freq_factor -> f; in between a linear blend with
    smooth = (old_ctx/wavelen - low) / (high - low).
    """
    f = 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))
    if not rope_scaling or rope_scaling.get("rope_type") != "llama3":
        return f
    factor = float(rope_scaling["factor"])
    low = float(rope_scaling["low_freq_factor"])
    high = float(rope_scaling["high_freq_factor"])
    old_ctx = float(rope_scaling["original_max_position_embeddings"])
    wavelen = 2 * math.pi / f
    scaled = torch.where(wavelen > old_ctx / low, f / factor, f)
    smooth = (old_ctx / wavelen - low) / (high - low)
    blended = (1 - smooth) * scaled / factor + smooth * scaled
    medium = (wavelen >= old_ctx / high) & (wavelen <= old_ctx / low)
    return torch.where(medium, blended, scaled)


def freqs_cis(dim: int, end: int, theta: float = 500000.0,
              rope_scaling: dict | None = None) -> torch.Tensor:
    """complex64 [end, dim/2] = exp(i * t * f) on CPU (src/rope.py:33-38)."""
    f = inv_freq(dim, theta, rope_scaling)
    ang = torch.outer(torch.arange(end), f).float()
    return torch.polar(torch.ones_like(ang), ang)


def cos_sin(fc: torch.Tensor, dtype: torch.dtype):
    """cos/sin rounded to the activation dtype (src/rope.py:41-45)."""
    return fc.real.to(dtype), fc.imag.to(dtype)


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE (src/rope.py:85-86) of x [..., S, D] with tables [S, D/2].

    Computed in fp32 from the stored values (each product and the sum rounded
    to fp32 separately), rounded once to x's dtype.
    """
    half = x.shape[-1] // 2
    xf = x.detach().to("cpu", torch.float32)
    c = cos.detach().to("cpu", torch.float32)
    s = sin.detach().to("cpu", torch.float32)
    x1, x2 = xf[..., :half], xf[..., half:]
    y1 = x1 * c - x2 * s
    y2 = x2 * c + x1 * s
    return torch.cat([y1, y2], dim=-1).to(x.dtype)


def kv_slot(layer: int, b: int, h: int, pos: int, d: int,
            max_batch: int, n_kv_heads: int, max_seq: int, head_dim: int) -> int:
    """Flat element index of cache[layer, b, h, pos, d] (src/kv_cache.py:15)."""
    return ((((layer * max_batch + b) * n_kv_heads + h) * max_seq + pos) * head_dim + d)


def rope_kv_append(cache_k: torch.Tensor, cache_v: torch.Tensor, layer: int,
                   xk: torch.Tensor, xv: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, start_pos: int | None = None,
                   positions: torch.Tensor | None = None):
    """Return copies of the caches after the fused K-RoPE + KV append.

    src/rope.py:122-252: for token s, pos = start_pos + s (:166) or
    positions[s] (:216), shared across the batch; cache_k[layer,b,h,pos] =
    RoPE(xk[b,h,s]) with cos/sin row s (:189-193), cache_v[...] = xv (bitwise).
    """
    ck = cache_k.detach().to("cpu").clone()
    cv = cache_v.detach().to("cpu").clone()
    B, H, S, D = xk.shape
    rk = rotate(xk, cos, sin).to(ck.dtype)
    pos = (torch.arange(S) + start_pos) if positions is None else positions.detach().to("cpu")
    for s in range(S):
        p = int(pos[s])
        ck[layer, :B, :, p] = rk[:, :, s]
        cv[layer, :B, :, p] = xv[:, :, s].detach().to("cpu", cv.dtype)
    return ck, cv
