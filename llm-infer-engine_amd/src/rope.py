"""Rotary position embedding (interface of src/rope.py in the reference).

Host-side table construction (``precompute_freqs_cis``/``build_rope_cos_sin``)
keeps the reference's CPU fp32 maths so tables match bit for bit; the per-token
work runs in HIP kernels:
  * ``apply_rotary``           -> mi_rope            (Q RoPE)
  * ``rope_and_cache_update``  -> mi_rope_kv_append  (K RoPE + KV-cache append,
                                  one launch, contiguous or scatter positions)
``DeviceRopeTable`` keeps a model's full cos/sin table resident in HBM so a
forward pass or a captured decode step never copies tables from the host.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def _compute_inv_freq(dim: int, theta: float, rope_scaling=None):
    """Inverse frequencies 1/theta^(2i/dim) in fp32, with optional llama3
    wavelength-based scaling (src/rope.py:8-30)."""
    base = 1.0 / (theta ** (torch.arange(0, dim, 2, device="cpu").float() / dim))
    if not rope_scaling or rope_scaling.get("rope_type") != "llama3":
        return base
    factor = float(rope_scaling["factor"])
    lo = float(rope_scaling["low_freq_factor"])
    hi = float(rope_scaling["high_freq_factor"])
    ctx = float(rope_scaling["original_max_position_embeddings"])
    wavelen = 2 * math.pi / base
    long_wave = wavelen > ctx / lo
    short_wave = wavelen < ctx / hi
    scaled = torch.where(long_wave, base / factor, base)
    t = (ctx / wavelen - lo) / (hi - lo)
    blend = (1 - t) * scaled / factor + t * scaled
    return torch.where(~short_wave & ~long_wave, blend, scaled)


def precompute_freqs_cis(dim: int, end: int, theta: float = 500000.0, rope_scaling=None):
    """complex64 [end, dim/2] table exp(i * pos * f) built on the CPU
    (src/rope.py:33-38)."""
    f = _compute_inv_freq(dim=dim, theta=theta, rope_scaling=rope_scaling)
    angles = torch.outer(torch.arange(end, device="cpu"), f).float()
    return torch.polar(torch.ones_like(angles), angles)


def build_rope_cos_sin(freqs_cis, dtype, device):
    """Half-length cos/sin [seq_len, head_dim // 2] in the activation dtype
    (src/rope.py:41-45)."""
    return (freqs_cis.real.to(device=device, dtype=dtype),
            freqs_cis.imag.to(device=device, dtype=dtype))


class DeviceRopeTable:
    """Full [max_seq_len, head_dim/2] cos/sin tables resident on the device.

    Built once from ``precompute_freqs_cis`` (so values equal the reference's
    per-forward tables); forwards take row slices (views, no copies) and the
    graph runner indexes rows by device-side positions.
    """

    def __init__(self, freqs_cis: torch.Tensor, dtype: torch.dtype, device):
        self.cos, self.sin = build_rope_cos_sin(freqs_cis, dtype, device)

    def rows(self, start: int, length: int):
        return self.cos[start:start + length], self.sin[start:start + length]


def _check_tables(cos: torch.Tensor, sin: torch.Tensor, seq_len: int, head_dim: int, what: str):
    if cos.dim() != 2 or sin.dim() != 2:
        raise ValueError(f"{what}: cos/sin must be 2-D [seq_len, head_dim // 2]")
    if cos.shape[1] < head_dim // 2 or sin.shape[1] < head_dim // 2:
        raise ValueError(f"{what}: cos/sin last dim must be head_dim // 2 = {head_dim // 2}")
    if cos.shape[0] < seq_len or sin.shape[0] < seq_len:
        raise ValueError(f"{what}: cos/sin have {cos.shape[0]} rows, need {seq_len}")
    if cos.dtype != sin.dtype:
        raise TypeError(f"{what}: cos and sin must share a dtype")


def apply_rotary(x, cos, sin, *, positions=None):
    """Rotate-half RoPE of x [B, n_heads, seq_len, head_dim] with cos/sin
    [seq_len, head_dim // 2]; returns a new tensor with x's strides
    (src/rope.py:94-119).  ``positions`` (keyword-only extension, device int64
    [seq_len]): cos/sin are full tables and token s uses row positions[s]
    (clamped into the table's rows)."""
    B, n_heads, seq_len, head_dim = x.shape
    _lib.require_device(x, "apply_rotary")
    _check_tables(cos, sin, seq_len if positions is None else 1, head_dim, "apply_rotary")
    if positions is not None and (positions.dtype != torch.int64 or positions.device != x.device):
        positions = positions.to(device=x.device, dtype=torch.int64)
    out = torch.empty_like(x)
    lib = _lib.load()
    st = lib.mi_rope(
        x.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(), _lib.ptr(positions),
        min(cos.shape[0], sin.shape[0]), B, n_heads, seq_len, head_dim,
        *x.stride(), *out.stride(), *cos.stride(), *sin.stride(),
        _lib.dtype_code(x.dtype), _lib.dtype_code(cos.dtype), _lib.stream_of(x))
    _lib.check(st, "apply_rotary")
    return out


def rope_and_cache_update(xk, xv, rope_cos, rope_sin, kv_cache, layer_idx,
                          start_pos=None, scatter_positions=None, *,
                          cos_by_position: bool = False):
    """Fused K RoPE + KV-cache write (src/rope.py:255-313).

    xk, xv: [B, n_kv_heads, S, head_dim]; token s goes to slot start_pos + s,
    or to scatter_positions[s] (a device tensor shared by the batch, the graph
    path).  Returns the cache views attention reads: [:, :, :start_pos+S] on the
    sequential path, the full [B, n_kv_heads, max_seq_len, head_dim] on the
    scatter path.  ``cos_by_position`` (keyword-only extension): rope_cos /
    rope_sin are full tables indexed by the absolute slot position.
    """
    B, n_kv_heads, input_len, head_dim = xk.shape
    if xv.shape != xk.shape:
        raise ValueError(f"xk and xv shapes must match, got {tuple(xk.shape)} and {tuple(xv.shape)}")
    # the kernel writes B x n_kv_heads x head_dim slabs of layer layer_idx: a
    # shape the cache does not hold would land in the next layer or past the end
    if (B > kv_cache.max_batch_size or n_kv_heads != kv_cache.n_kv_heads
            or head_dim != kv_cache.head_dim):
        raise ValueError(f"xk/xv shape {tuple(xk.shape)} does not fit the cache "
                         f"[{kv_cache.max_batch_size}, {kv_cache.n_kv_heads}, *, {kv_cache.head_dim}]")
    if not -kv_cache.k.shape[0] <= layer_idx < kv_cache.k.shape[0]:
        raise ValueError(f"layer_idx {layer_idx} out of range for a cache of {kv_cache.k.shape[0]} layers")
    _lib.require_device(xk, "rope_and_cache_update")
    if scatter_positions is None and start_pos is None:
        raise ValueError("rope_and_cache_update needs start_pos or scatter_positions")
    _check_tables(rope_cos, rope_sin, 1 if cos_by_position else input_len, head_dim,
                  "rope_and_cache_update")
    cache_k = kv_cache.k[layer_idx, :B]
    cache_v = kv_cache.v[layer_idx, :B]
    if xk.dtype != cache_k.dtype or xv.dtype != cache_v.dtype:
        raise TypeError(f"xk/xv dtype {xk.dtype} must match the cache dtype {cache_k.dtype}")
    positions = None
    if scatter_positions is not None:
        if scatter_positions.dim() != 1 or scatter_positions.shape[0] < input_len:
            raise ValueError("scatter_positions must be 1-D with one entry per token")
        positions = scatter_positions
        if positions.dtype != torch.int64 or positions.device != xk.device:
            positions = positions.to(device=xk.device, dtype=torch.int64)
    lib = _lib.load()
    st = lib.mi_rope_kv_append(
        xk.data_ptr(), xv.data_ptr(), rope_cos.data_ptr(), rope_sin.data_ptr(),
        cache_k.data_ptr(), cache_v.data_ptr(),
        0 if start_pos is None else int(start_pos), _lib.ptr(positions),
        min(rope_cos.shape[0], rope_sin.shape[0]), B, n_kv_heads, input_len, head_dim, cache_k.shape[2],
        *xk.stride(), *xv.stride(), *cache_k.stride(), *cache_v.stride(),
        *rope_cos.stride(), *rope_sin.stride(), int(bool(cos_by_position)),
        _lib.dtype_code(xk.dtype), _lib.dtype_code(rope_cos.dtype), _lib.stream_of(xk))
    _lib.check(st, "rope_and_cache_update")
    if scatter_positions is not None:
        return cache_k, cache_v
    end_pos = int(start_pos) + input_len
    return cache_k[:, :, :end_pos], cache_v[:, :, :end_pos]
