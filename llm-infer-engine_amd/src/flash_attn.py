"""Causal GQA flash-attention prefill (interface of src/flash_attn.py).

``flash_attention(q, k, v)`` keeps the reference signature and semantics
(src/flash_attn.py:85-111): q [B, Hq, S, D], k/v [B, Hkv, L, D]; query head h
reads kv head h // (Hq // Hkv); query row i attends keys 0..i of the first S
keys; out has q's dtype and strides.  The GQA expand/reshape copy of the
reference (src/flash_attn.py:92-94) is gone: the HIP kernel stages each K/V tile
once in LDS for all query heads of a group.  Keyword-only extensions:
  return_lse  also return lse [B, Hq, S] fp32 (natural log of scaled scores)
  sm_scale    softmax scale (default 1/sqrt(D), as the reference)
  rope_cos, rope_sin, rope_positions
              apply the rotate-half RoPE of apply_rotary (src/rope.py) to q
              first: flash_attention(q, k, v, rope_cos=c, rope_sin=s) gives the
              bits of flash_attention(apply_rotary(q, c, s), k, v).  With tables
              in q's dtype the rotation runs in the attention kernel's Q prologue
              (one launch, q never rewritten); otherwise apply_rotary runs first.
head_dim 16, 32, 64, 128 or 256 (src/flash_attn.py:29-32 takes any power of
two): bf16/fp16 at 32 to 256 run on MFMA, head_dim 16 and fp32 on a VALU
kernel in fp32 arithmetic.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def _ready(t: torch.Tensor) -> torch.Tensor:
    es = t.element_size()
    if (t.stride(3) == 1 and t.data_ptr() % 16 == 0
            and all((s * es) % 16 == 0 for s in t.stride()[:3])):
        return t
    return t.contiguous()


def flash_attention(q, k, v, *, return_lse: bool = False, sm_scale: float | None = None,
                    rope_cos=None, rope_sin=None, rope_positions=None):
    # expect q: [batch, n_heads, seq_len, head_dim]
    # expect k,v: [batch, n_kv_heads, kv_seq_len >= seq_len, head_dim]
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must all be rank-4 tensors")
    batch_size, n_heads, seq_len, head_dim = q.shape
    kb, n_kv_heads, kv_seq_len, kd = k.shape
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes must match, got {k.shape} and {v.shape}")
    if kb != batch_size or kd != head_dim:
        raise ValueError("q and k/v batch size and head dimension must match")
    if n_heads % n_kv_heads != 0:
        raise ValueError(f"query heads ({n_heads}) must be divisible by KV heads ({n_kv_heads})")
    if kv_seq_len < seq_len:
        raise ValueError(f"k/v hold {kv_seq_len} positions, fewer than the {seq_len} queries")
    _lib.require_device(q, "flash_attention")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, and v must have the same dtype")
    rope = rope_cos is not None or rope_sin is not None
    if rope:
        from .rope import _check_tables, apply_rotary
        if rope_cos is None or rope_sin is None:
            raise ValueError("flash_attention: rope_cos and rope_sin go together")
        if rope_positions is None:
            _check_tables(rope_cos, rope_sin, seq_len, head_dim, "flash_attention")
        elif rope_positions.numel() < seq_len:
            raise ValueError(f"flash_attention: {rope_positions.numel()} rope positions for "
                             f"{seq_len} queries")
        fuse = (rope_cos.dtype == q.dtype and rope_cos.shape == rope_sin.shape
                and rope_cos.stride() == rope_sin.stride()
                and rope_cos.dim() == 2 and rope_cos.stride(1) == 1
                and rope_cos.shape[1] >= head_dim // 2
                and (q.dtype == torch.float32
                     or ((rope_cos.stride(0) * 2) % 16 == 0
                         and rope_cos.data_ptr() % 16 == 0 and rope_sin.data_ptr() % 16 == 0)))
        if not fuse:
            q = apply_rotary(q, rope_cos, rope_sin, positions=rope_positions)
            rope = False
        elif rope_positions is not None and (rope_positions.dtype != torch.int64
                                             or rope_positions.device != q.device):
            rope_positions = rope_positions.to(device=q.device, dtype=torch.int64)
    q_, k_, v_ = _ready(q), _ready(k), _ready(v)
    out = torch.empty_like(q)
    o_ = out if (out.stride(3) == 1 and out.data_ptr() % 16 == 0) else torch.empty(
        q.shape, dtype=q.dtype, device=q.device)
    lse = (torch.empty((batch_size, n_heads, seq_len), device=q.device, dtype=torch.float32)
           if return_lse else None)
    scale = (1.0 / math.sqrt(head_dim)) if sm_scale is None else float(sm_scale)
    if seq_len > 0:
        lib = _lib.load()
        common = (q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o_.data_ptr(), _lib.ptr(lse),
                  batch_size, n_heads, n_kv_heads, seq_len, kv_seq_len, head_dim,
                  q_.stride(0), q_.stride(1), q_.stride(2),
                  k_.stride(0), k_.stride(1), k_.stride(2),
                  v_.stride(0), v_.stride(1), v_.stride(2),
                  o_.stride(0), o_.stride(1), o_.stride(2), scale)
        if rope:
            st = lib.mi_attn_prefill_rope(
                *common, rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.shape[0],
                rope_cos.stride(0), _lib.ptr(rope_positions), _lib.dtype_code(q.dtype),
                _lib.stream_of(q))
        else:
            st = lib.mi_attn_prefill(*common, _lib.dtype_code(q.dtype), _lib.stream_of(q))
        _lib.check(st, "flash_attention")
    if o_ is not out:
        out.copy_(o_)
    return (out, lse) if return_lse else out
