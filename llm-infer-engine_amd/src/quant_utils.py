"""Symmetric per-channel int8 weight quantisation (interface of
src/quant_utils.py:7-36), run by one HIP launch (mi_quantize_int8):

    amax  = max(max_k |w[n, k]|, 1e-12)            in fp32
    scale = (amax / 127) rounded to w's dtype        [N, 1]
    q     = clamp(round_half_even(w / scale), -128, 127) as int8

Each step is a correctly rounded IEEE operation, so q and scale are bit-exact
with the reference's torch recipe.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib


def quantize_weight_symmetric_per_channel(
    weight: torch.Tensor,
    quant_dtype: torch.dtype = torch.int8,
) -> Tuple[torch.Tensor, torch.Tensor]:
    orig_dtype = weight.dtype
    if orig_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"Unsupported weight dtype for quantization: {orig_dtype}")
    if quant_dtype != torch.int8:
        raise NotImplementedError("Only int8 symmetric per-channel quantization is supported.")
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [out_features, in_features], got {tuple(weight.shape)}")
    _lib.require_device(weight, "quantize_weight_symmetric_per_channel")
    w = weight if weight.stride(1) == 1 else weight.contiguous()
    N, K = w.shape
    qweight = torch.empty((N, K), dtype=torch.int8, device=w.device)
    scales = torch.empty((N, 1), dtype=orig_dtype, device=w.device)
    st = _lib.load().mi_quantize_int8(
        w.data_ptr(), qweight.data_ptr(), scales.data_ptr(), N, K, w.stride(0),
        qweight.stride(0), _lib.dtype_code(orig_dtype), _lib.stream_of(w))
    _lib.check(st, "quantize_weight_symmetric_per_channel")
    return qweight, scales


# ---------------------------------------------------------------------------
# Which state-dict keys are quantised, and the accuracy metrics used to compare
# a W8A16 model with its bf16 master (src/quant_utils.py:39-121).

def get_transformer_linear_names() -> Tuple[str, ...]:
    """Module paths (below "layers.{i}.") of the seven W8A16 projections."""
    return ("attention.wq", "attention.wk", "attention.wv", "attention.wo",
            "feed_forward.w1", "feed_forward.w2", "feed_forward.w3")


def should_quantize_key(model_key: str) -> bool:
    """True for "layers.{i}.<projection>.weight" keys of the seven projections."""
    parts = model_key.split(".")
    if len(parts) < 5 or parts[0] != "layers" or parts[-1] != "weight":
        return False
    return ".".join(parts[2:-1]) in get_transformer_linear_names()


# Accuracy metrics comparing a W8A16 model's logits with its bf16 master (the
# reference's evaluation scripts import them, src/quant_utils.py:39-96); plain
# torch reductions, not on the hot path.

def cosine_similarity(a: torch.Tensor, b: torch.Tensor, eps: float = 1e-12) -> torch.Tensor:
    """Mean over rows (all leading dims) of cos(a_row, b_row), in fp32."""
    a2 = a.reshape(-1, a.shape[-1]).float()
    b2 = b.reshape(-1, b.shape[-1]).float()
    dots = (a2 * b2).sum(dim=1)
    norms = (a2.norm(dim=1) * b2.norm(dim=1)).clamp_min(eps)
    return (dots / norms).mean()


def logits_max_abs_error(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).abs().max())


def logits_relative_error(a: torch.Tensor, b: torch.Tensor, eps: float = 1e-12) -> float:
    """Mean of |a - b| / max(|a|, eps) over elements (a is the reference)."""
    af = a.float()
    return float(((af - b.float()).abs() / af.abs().clamp_min(eps)).mean())


def top1_agreement(a: torch.Tensor, b: torch.Tensor) -> float:
    """Fraction of positions whose argmax over the last dim agrees."""
    return float((a.argmax(dim=-1) == b.argmax(dim=-1)).float().mean())


def perplexity(logits: torch.Tensor, labels: torch.Tensor) -> float:
    """exp(mean next-token cross entropy): logits[:, t] predicts labels[:, t+1];
    [S, V] / [S] inputs are treated as one sequence; labels == -100 are ignored."""
    if logits.dim() == 2:
        logits, labels = logits[None], labels[None]
    pred = logits[:, :-1, :].float().reshape(-1, logits.shape[-1])
    tgt = labels[:, 1:].reshape(-1)
    nll = torch.nn.functional.cross_entropy(pred, tgt, reduction="mean", ignore_index=-100)
    return float(torch.exp(nll))
