"""W8A16 Llama-3 module tree (interface of src/model_quantized.py).

Same composition as src/model.py with W8A16Linear for the seven per-layer
projections; embedding, norms and lm_head stay in the activation dtype
(src/model_quantized.py:137-142).  ``build_random_quantized`` makes the seeded
random-init model of the W8A16 decode benchmark: bf16 master weights drawn on
the device, quantised with quantize_weight_symmetric_per_channel.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .model import Attention, FeedForward, Llama3, TransformerBlock
from .quant_linear import W8A16Linear
from .quant_utils import quantize_weight_symmetric_per_channel


class QuantizedFeedForward(FeedForward):
    def __init__(self, dim: int, hidden_dim: int):
        super().__init__(dim, hidden_dim, W8A16Linear)


class QuantizedAttention(Attention):
    def __init__(self, args):
        super().__init__(args, W8A16Linear)


class QuantizedTransformerBlock(TransformerBlock):
    def __init__(self, args, linear=W8A16Linear):
        super().__init__(args, W8A16Linear)


class Llama3Quantized(Llama3):
    block_cls = QuantizedTransformerBlock
    linear_cls = W8A16Linear


_QUANT_NAMES = ("attention.wq", "attention.wk", "attention.wv", "attention.wo",
                "feed_forward.w1", "feed_forward.w2", "feed_forward.w3")


@torch.no_grad()
def build_random_quantized(args, seed: int = 0, dtype=torch.bfloat16, device="cuda") -> Llama3Quantized:
    """Seeded random-init W8A16 model on `device`.

    Master weights: linears ~ U(-1/sqrt(in), 1/sqrt(in)) (nn.Linear's default
    range), embedding ~ N(0, 1), norms = 1, all in `dtype`; each per-layer
    linear is then quantised with the symmetric per-channel int8 recipe.
    """
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.device("meta"):
        model = Llama3Quantized(args)
    model = model.to_empty(device=device)
    model.tok_embeddings.weight.data = torch.randn(
        model.tok_embeddings.weight.shape, generator=g, device=device, dtype=torch.float32).to(dtype)
    bound = 1.0 / (args.dim ** 0.5)
    model.output.weight.data = ((torch.rand(model.output.weight.shape, generator=g, device=device,
                                            dtype=torch.float32) * 2 - 1) * bound).to(dtype)
    for layer in model.layers:
        for name in _QUANT_NAMES:
            mod = layer.get_submodule(name)
            b = 1.0 / (mod.in_features ** 0.5)
            w = ((torch.rand((mod.out_features, mod.in_features), generator=g, device=device,
                             dtype=torch.float32) * 2 - 1) * b).to(dtype)
            q, s = quantize_weight_symmetric_per_channel(w)
            mod.weight.data = q
            mod.scales.data = s
        layer.attention_norm.weight.data = torch.ones(args.dim, device=device, dtype=dtype)
        layer.ffn_norm.weight.data = torch.ones(args.dim, device=device, dtype=dtype)
    model.norm.weight.data = torch.ones(args.dim, device=device, dtype=dtype)
    return model.eval()
