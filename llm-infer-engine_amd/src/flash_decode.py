"""Split-KV flash decode (interface of src/flash_decode.py in the reference).

``flash_decode(q, k, v, mask=None)`` keeps the reference's signature, argument
checks and error messages (src/flash_decode.py:215-285) and the same result:
softmax over the keys j < L with mask[b, j] true, 0 for a row with no such key.
The work runs in one HIP launch (mi_flash_decode): a split kernel whose
workgroups each stream one (batch, kv-head, key-range) ONCE for all query heads
of the GQA group, and whose last workgroup of each group combines the group's
partials (LSE combine) from its XCD's L2.  Keyword-only extensions:
  num_splits  key-range count (default: chosen from the CU count); there is no
              65,536-key cap as in the reference (src/flash_decode.py:278-279).
  seq_lens    int64 [B] device tensor; keys >= seq_lens[b] are never read
              (graph-safe variable lengths without a mask).
  return_lse  also return the fp32 log-sum-exp [B, Hq] of the scaled scores.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def _mask_strides(mask: torch.Tensor, batch_size: int, kv_len: int) -> tuple[int, int]:
    """Validate a bool mask of shape [L'], [B|1, L'] or [B|1, 1, ..., L'] with
    L' >= kv_len and return its (batch, key) element strides (batch stride 0 =
    broadcast) — same rules and messages as src/flash_decode.py:215-233."""
    if mask.dtype != torch.bool:
        raise TypeError(f"mask must have dtype torch.bool, got {mask.dtype}")
    if mask.ndim == 0:
        raise ValueError("mask must have at least one dimension")
    if mask.ndim == 1:
        if mask.shape[0] < kv_len:
            raise ValueError("mask is shorter than the KV sequence")
        return 0, mask.stride(0)
    if mask.shape[0] not in (1, batch_size):
        raise ValueError(f"mask batch dimension must be 1 or {batch_size}, got {mask.shape[0]}")
    if any(size != 1 for size in mask.shape[1:-1]):
        raise ValueError("all mask dimensions except batch and KV length must be 1")
    if mask.shape[-1] < kv_len:
        raise ValueError("mask is shorter than the KV sequence")
    return (0 if mask.shape[0] == 1 else mask.stride(0), mask.stride(-1))


def _kv_ready(t: torch.Tensor) -> torch.Tensor:
    """K/V rows must have unit innermost stride (rows that are also 16-byte
    aligned are read with 128-bit loads, others element by element); other
    layouts are re-laid out once (a copy, not compute)."""
    if t.stride(3) == 1 or t.shape[3] == 1:
        return t
    return t.contiguous()


def default_num_splits(batch: int, n_heads: int, n_kv_heads: int, kv_len: int,
                       head_dim: int) -> int:
    return int(_lib.load().mi_decode_default_splits(batch, n_heads, n_kv_heads, kv_len, head_dim))


def _run_decode(q, k, v, mask, seq_lens, num_splits, return_lse, empty_nan, what):
    batch_size, n_heads, _, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    mask_sb = mask_sl = 0
    if mask is not None:
        if not mask.is_cuda or mask.device != q.device:
            raise ValueError("mask must be on the same CUDA device as q")
        mask_sb, mask_sl = _mask_strides(mask, batch_size, kv_len)
    if seq_lens is not None:
        if seq_lens.shape != (batch_size,):
            raise ValueError(f"seq_lens must have shape ({batch_size},), got {tuple(seq_lens.shape)}")
        if seq_lens.device != q.device or seq_lens.dtype != torch.int64:
            seq_lens = seq_lens.to(device=q.device, dtype=torch.int64)
    if num_splits is None:
        num_splits = default_num_splits(batch_size, n_heads, n_kv_heads, kv_len, head_dim)
    num_splits = int(num_splits)
    if num_splits < 1:
        raise ValueError(f"num_splits must be >= 1, got {num_splits}")
    num_splits = min(num_splits, kv_len)
    # too few splits to fill the GPU are subdivided into >= 1024-key ranges
    num_splits = int(_lib.load().mi_decode_effective_splits(
        batch_size, n_heads, n_kv_heads, kv_len, head_dim, num_splits))
    k = _kv_ready(k)
    v = _kv_ready(v)
    out = torch.empty_like(q)
    lse = torch.empty((batch_size, n_heads), device=q.device, dtype=torch.float32) if return_lse else None
    if num_splits > 1:
        part_m = torch.empty((batch_size, n_heads, num_splits), device=q.device, dtype=torch.float32)
        part_l = torch.empty_like(part_m)
        part_acc = torch.empty((batch_size, n_heads, num_splits, head_dim),
                               device=q.device, dtype=torch.float32)
    else:
        part_m = part_l = part_acc = None
    lib = _lib.load()
    # with several splits the LSE combine runs inside the split launch, on the
    # library's per-stream arrival counters (batch * n_heads bounds the groups)
    arrive = _lib.arrive_counters(q, batch_size * n_heads) if num_splits > 1 else None
    st = lib.mi_flash_decode(
        q.data_ptr(), k.data_ptr(), v.data_ptr(),
        _lib.ptr(mask), mask_sb, mask_sl, _lib.ptr(seq_lens),
        _lib.ptr(part_m), _lib.ptr(part_l), _lib.ptr(part_acc), arrive,
        out.data_ptr(), _lib.ptr(lse),
        batch_size, n_heads, n_kv_heads, kv_len, head_dim, num_splits,
        q.stride(0), q.stride(1), q.stride(3),
        k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2),
        out.stride(0), out.stride(1), out.stride(3),
        1.0 / math.sqrt(head_dim), int(empty_nan), _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(st, what)
    return (out, lse) if return_lse else out


def flash_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: torch.Tensor | None = None,
    *,
    num_splits: int | None = None,
    seq_lens: torch.Tensor | None = None,
    return_lse: bool = False,
):
    """Single-token GQA/MQA attention with split-KV parallelism.

    Shapes are q=[B, Hq, 1, D] and k/v=[B, Hkv, L, D]. A boolean mask may
    have shape [L], [B, L], or [B, 1, 1, L].
    """
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must all be rank-4 tensors")
    batch_size, n_heads, query_len, head_dim = q.shape
    k_batch, n_kv_heads, kv_len, k_head_dim = k.shape
    if query_len != 1:
        raise ValueError(f"flash_decode only supports query_len=1, got {query_len}")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes must match, got {k.shape} and {v.shape}")
    if k_batch != batch_size or k_head_dim != head_dim:
        raise ValueError("q and k/v batch size and head dimension must match")
    if kv_len == 0:
        raise ValueError("KV sequence must not be empty")
    if n_heads % n_kv_heads != 0:
        raise ValueError(f"query heads ({n_heads}) must be divisible by KV heads ({n_kv_heads})")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("flash_decode requires CUDA tensors")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, and v must be on the same device")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, and v must have the same dtype")
    if head_dim > 256:
        raise ValueError(f"head_dim must be <= 256, got {head_dim}")
    return _run_decode(q, k, v, mask, seq_lens, num_splits, return_lse, False, "flash_decode")


# Keep the attention-style name convenient for callers (src/flash_decode.py:374).
flash_decode_attention = flash_decode
