"""numpy/torch CPU restatement of the quantiser, W8A16 linear and RMSNorm.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np
import torch


def _round_f32_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to bf16 / fp16 (round-to-nearest-even), returned as fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        u = x.view(np.uint32).astype(np.uint64)
        lsb = (u >> 16) & 1
        r = ((u + 0x7FFF + lsb) >> 16) << 16
        nan = np.isnan(x)
        out = r.astype(np.uint32).view(np.float32).copy()
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def quantize_per_channel(w: np.ndarray, dtype: str):
    """Symmetric per-channel int8 quantisation (src/quant_utils.py:28-35).

    w: [N, K] fp32 holding values of `dtype`.  amax = max(max_k |w|, 1e-12)
    (:30-32); scale = round_to_dtype(amax / 127) (:34); q = clamp(rint(w /
    scale), -128, 127) (:35), the division in fp32 and rint = half-to-even.
    Returns (q int8 [N, K], scale fp32 [N, 1] holding dtype values).
    """
    w = np.asarray(w, dtype=np.float32)
    amax = np.maximum(np.abs(w).max(axis=1, keepdims=True), np.float32(1e-12)).astype(np.float32)
    scale = _round_f32_to(amax / np.float32(127.0), dtype)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(w / scale)
    # 0/0 (all-zero fp16 row, scale underflow) is NaN in the recipe; its int8
    # cast is platform-defined there (0 on x86 torch): pinned to 0 here.
    q = np.clip(np.nan_to_num(r, nan=0.0), -128, 127).astype(np.int8)
    return q, scale


def w8a16(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """fp32 dequant matmul, the reference test's reference (tests/quant_unit.py:64-77):
    (x.f32 @ (q.f32 * s.f32)^T), rounded to x's dtype."""
    xf = x.detach().to("cpu", torch.float32)
    wd = q.detach().to("cpu", torch.float32) * s.detach().to("cpu", torch.float32).reshape(-1, 1)
    return (xf @ wd.t()).to(x.dtype)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w in fp32, stored in x's dtype
    (src/rms_norm.py:32-38)."""
    xf = x.detach().to("cpu", torch.float32)
    wf = w.detach().to("cpu", torch.float32)
    r = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
    return (xf * r * wf).to(x.dtype)
