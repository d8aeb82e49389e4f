"""Fused W8A16 decode-step ops (one token per row, up to 16 rows).

A decode step of the W8A16 block (src/model_quantized.py:42-93, the block
composition of src/model.py:93-127) runs here in six launches per layer
instead of one per reference op:

  qkv_rope_append   rmsnorm -> wq|wk|wv -> RoPE(q); RoPE(k), v -> KV cache
  flash_decode      split-KV attention over the cache and its LSE combine
                    (two launches, src/flash_decode.py)
  linear_fused      wo + residual;  rmsnorm -> w1|w3 -> silu*mul;  w2 + residual

Every value is rounded where the reference's separate ops round it (see
include/miattn.h), so the fused step equals the unfused composition up to
fp32 summation order.  These are the HIP kernels of libmiattn.so; there is no
other implementation.
"""
from __future__ import annotations

import torch

from . import _lib

EPI_STORE = 0
EPI_RESIDUAL = 1
EPI_SWIGLU = 2


def _w(lin):
    """int8 weight [N, K], scales [N] of a W8A16Linear."""
    return lin.weight, lin.scales.reshape(-1)


#: reduction lengths the fused GEMV kernels are built for (K = 512 * waves)
SUPPORTED_K = (512, 1024, 1536, 2048, 3072, 4096, 6144, 8192)


def supported(M: int, K: int, dtype: torch.dtype, lin, norm_weight=None, *,
              swiglu: bool = False) -> bool:
    """Whether the fused kernels take an [M, K] input of `dtype` through W8A16
    layer `lin` (and RMSNorm weight `norm_weight`); the input itself must also
    be row-aligned (``aligned``).  Otherwise use the op-by-op path."""
    if dtype not in (torch.bfloat16, torch.float16):
        return False
    w, s = _w(lin)
    if not (1 <= M <= 16 and K in SUPPORTED_K and w.dtype == torch.int8):
        return False
    if not (w.is_contiguous() and w.shape[1] == K and w.data_ptr() % 16 == 0):
        return False
    if s.dtype != dtype or not s.is_contiguous():
        return False
    if swiglu and K > 4096:
        return False
    if norm_weight is not None:
        if (norm_weight.dtype != dtype or not norm_weight.is_contiguous()
                or norm_weight.data_ptr() % 16 != 0 or M * K * 2 > 64 * 1024
                or (M > 8 and K > 2048)):
            return False
    return True


def aligned(x: torch.Tensor) -> bool:
    """Rows of x [M, K] are unit-stride and 16-byte aligned."""
    return (x.is_cuda and x.stride(1) == 1 and x.data_ptr() % 16 == 0
            and (x.stride(0) * x.element_size()) % 16 == 0)


def linear_fused(x, lin, *, norm_weight=None, eps: float = 0.0, lin_b=None, residual=None):
    """y = epilogue(W8A16(rmsnorm?(x))) for x [M, K]; returns [M, N].

    residual [M, N]: y = residual + linear;  lin_b: y = silu(lin(x)) * lin_b(x).
    """
    M, K = x.shape
    w, s = _w(lin)
    N = w.shape[0]
    y = torch.empty((M, N), device=x.device, dtype=x.dtype)
    if lin_b is not None:
        wb, sb = _w(lin_b)
        epi = EPI_SWIGLU
    else:
        wb, sb = None, None
        epi = EPI_RESIDUAL if residual is not None else EPI_STORE
    st = _lib.load().mi_w8a16_linear_fused(
        x.data_ptr(), x.stride(0), _lib.ptr(norm_weight), float(eps),
        w.data_ptr(), s.data_ptr(), w.stride(0),
        _lib.ptr(wb), _lib.ptr(sb), 0 if wb is None else wb.stride(0),
        _lib.ptr(residual), 0 if residual is None else residual.stride(0),
        y.data_ptr(), y.stride(0), M, N, K, epi, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_linear_fused")
    return y


def qkv_rope_append(x, attn, norm_weight, eps, rope_cos, rope_sin, rope_row0: int,
                    pos: torch.Tensor, kv_cache, layer_idx: int):
    """rmsnorm -> wq|wk|wv -> RoPE; writes RoPE(k), v into cache slot pos[0] of
    layer `layer_idx` for rows 0..M-1 and returns q [M, n_heads, 1, head_dim].

    rope_cos/rope_sin [rows, head_dim/2]; position p uses row p - rope_row0.
    """
    M, K = x.shape
    Hq, Hkv, D = attn.n_heads, attn.n_kv_heads, attn.head_dim
    wq, sq = _w(attn.wq)
    wk, sk = _w(attn.wk)
    wv, sv = _w(attn.wv)
    ck = kv_cache.k[layer_idx, :M]
    cv = kv_cache.v[layer_idx, :M]
    if ck.dtype != x.dtype or rope_cos.dtype != x.dtype or rope_cos.stride() != rope_sin.stride():
        raise TypeError("fused QKV: cache, rope tables and activations must share a dtype and layout")
    q = torch.empty((M, Hq, 1, D), device=x.device, dtype=x.dtype)
    st = _lib.load().mi_w8a16_qkv_rope_append(
        x.data_ptr(), x.stride(0), _lib.ptr(norm_weight), float(eps),
        wq.data_ptr(), sq.data_ptr(), wq.stride(0), wk.data_ptr(), sk.data_ptr(), wk.stride(0),
        wv.data_ptr(), sv.data_ptr(), wv.stride(0),
        rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.stride(0), int(rope_row0),
        rope_cos.shape[0], pos.data_ptr(), q.data_ptr(), ck.data_ptr(), cv.data_ptr(),
        ck.stride(0), ck.stride(1), ck.stride(2), ck.shape[2],
        M, K, Hq, Hkv, D, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_qkv_rope_append")
    return q
