"""W8A16 Llama-3 module tree (interface of src/model_quantized.py).

Same composition as src/model.py with W8A16Linear for the seven per-layer
projections; embedding, norms and lm_head stay in the activation dtype
(src/model_quantized.py:137-142).  ``build_random_quantized`` makes the seeded
random-init model of the W8A16 decode benchmark: bf16 master weights drawn on
the device, quantised with quantize_weight_symmetric_per_channel.

Single-token decode (query length 1, up to 16 rows) runs each block through
the fused decode-layer kernels (src/decode_layer.py): six launches per layer
with the same rounding points as the op-by-op composition.  Prefill-sized
inputs keep the composition but fuse its GEMMs: wq|wk|wv in one launch
(QuantizedAttention.qkv), silu(w1(x)) * w3(x) in one launch
(QuantizedFeedForward), and the block's residual adds in the wo / w2
epilogues; other shapes run op by op.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import decode_layer, quant_linear
from .flash_decode import flash_decode
from .model import Attention, FeedForward, Llama3, TransformerBlock
from .quant_linear import W8A16Linear
from .quant_utils import quantize_weight_symmetric_per_channel


class QuantizedFeedForward(FeedForward):
    def __init__(self, dim: int, hidden_dim: int, linear=W8A16Linear):
        super().__init__(dim, hidden_dim, linear)

    def forward(self, x, *, residual=None):
        """Prefill-sized inputs: silu(w1(x)) * w3(x) in one GEMM launch (the
        same rounding points, neither projection written out) when its tiles
        fill the GPU; otherwise the op chain of src/model.py:23."""
        x2 = x.reshape(-1, x.shape[-1])
        w1, w3 = self.w1, self.w3
        if not quant_linear.swiglu_worth(x2.shape[0], x2.shape[1], w1.out_features, x.device):
            return super().forward(x, residual=residual)
        torch.cuda.nvtx.range_push("FFN")
        h = quant_linear.w8a16_gemm_swiglu(x2, w1.weight, w1.scales, w3.weight, w3.scales)
        out = self.down(h.view(*x.shape[:-1], w1.out_features), residual)
        torch.cuda.nvtx.range_pop()
        return out

    def down(self, h, residual=None):
        return _project_residual(self.w2, h, residual)


def _project_residual(lin, h, residual):
    """lin(h) + residual with the add in the GEMM epilogue at GEMM sizes (the
    same roundings as the separate ops); otherwise the two ops."""
    h2 = h.reshape(-1, h.shape[-1])
    if residual is None or not quant_linear.gemm_supported(h2.shape[0], h2.shape[1]):
        out = lin(h)
        return out if residual is None else residual + out
    res2 = residual.reshape(-1, lin.out_features)
    y = quant_linear.w8a16_gemm_residual(h2, lin.weight, lin.scales, res2)
    return y.view(*h.shape[:-1], lin.out_features)


class QuantizedAttention(Attention):
    def __init__(self, args, linear=W8A16Linear):
        super().__init__(args, linear)

    def out_proj(self, output, residual=None):
        return _project_residual(self.wo, output, residual)

    def qkv(self, x):
        """Prefill-sized inputs: wq, wk and wv in one GEMM launch (bitwise the
        three separate GEMMs without a K split) when their tiles together
        fill the GPU; otherwise one W8A16Linear call each."""
        x2 = x.reshape(-1, x.shape[-1])
        mats = (self.wq, self.wk, self.wv)
        if not quant_linear.gemm_multi_worth(x2.shape[0], x2.shape[1],
                                             [m.out_features for m in mats], x.device):
            return super().qkv(x)
        ys = quant_linear.w8a16_gemm_multi(x2, [(m.weight, m.scales) for m in mats])
        return tuple(y.reshape(*x.shape[:-1], m.out_features) for y, m in zip(ys, mats))


class QuantizedTransformerBlock(TransformerBlock):
    #: run single-token decode through the fused decode-layer kernels
    fused_decode = True
    #: prefill-sized inputs: q|k|v in one GEMM launch, wo / w2 with the
    #: residual add in their epilogues, silu(w1) * w3 in one launch
    attention_cls = QuantizedAttention
    feed_forward_cls = QuantizedFeedForward

    def __init__(self, args, linear=W8A16Linear):
        super().__init__(args, W8A16Linear)

    def _fusable(self, x, rope_cos, kv_cache, layer_idx, positions, rope_by_position) -> bool:
        if not self.fused_decode or kv_cache is None or layer_idx is None or x.shape[1] != 1:
            return False
        if positions is not None and not rope_by_position:
            return False  # per-step sliced tables at a device position: op chain
        attn, ff = self.attention, self.feed_forward
        B, _, dim = x.shape
        if (B > kv_cache.max_batch_size or kv_cache.k.dtype != x.dtype
                or rope_cos.dtype != x.dtype or attn.head_dim % 16 != 0 or not x.is_contiguous()):
            return False
        dt, sup = x.dtype, decode_layer.supported
        n_o = attn.n_heads * attn.head_dim
        return (decode_layer.aligned(x.view(B, dim))
                and sup(B, dim, dt, attn.wq, self.attention_norm.weight)
                and sup(B, dim, dt, attn.wk) and sup(B, dim, dt, attn.wv)
                and sup(B, n_o, dt, attn.wo)
                and sup(B, dim, dt, ff.w1, self.ffn_norm.weight, swiglu=True)
                and sup(B, dim, dt, ff.w3)
                and sup(B, ff.w1.out_features, dt, ff.w2))

    def forward(self, x, rope_cos, rope_sin, layer_idx=None, start_pos=0, kv_cache=None,
                use_cuda_graph=False, scatter_positions=None, decode_attn_mask=None, **ext):
        positions = scatter_positions if (use_cuda_graph and scatter_positions is not None) else None
        by_pos = bool(ext.get("rope_by_position", False))
        if not self._fusable(x, rope_cos, kv_cache, layer_idx, positions, by_pos):
            return super().forward(x, rope_cos, rope_sin, layer_idx=layer_idx, start_pos=start_pos,
                                   kv_cache=kv_cache, use_cuda_graph=use_cuda_graph,
                                   scatter_positions=scatter_positions,
                                   decode_attn_mask=decode_attn_mask, **ext)
        attn, ff = self.attention, self.feed_forward
        B, _, dim = x.shape
        x2 = x.view(B, dim)
        if positions is not None:  # graph path: device position, full-table RoPE rows
            pos, row0 = positions, 0
            if pos.dtype != torch.int64:
                pos = pos.to(torch.int64)
        else:
            pos = torch.full((1,), int(start_pos), dtype=torch.int64, device=x.device)
            row0 = 0 if by_pos else int(start_pos)
        q = decode_layer.qkv_rope_append(x2, attn, self.attention_norm.weight,
                                         self.attention_norm.eps, rope_cos, rope_sin, row0, pos,
                                         kv_cache, layer_idx)
        ck, cv = kv_cache.k[layer_idx, :B], kv_cache.v[layer_idx, :B]
        if positions is None:
            ck, cv = ck[:, :, :int(start_pos) + 1], cv[:, :, :int(start_pos) + 1]
        o = flash_decode(q, ck, cv, mask=decode_attn_mask, seq_lens=ext.get("seq_lens"))
        h = decode_layer.linear_fused(o.view(B, -1), attn.wo, residual=x2)
        g = decode_layer.linear_fused(h, ff.w1, norm_weight=self.ffn_norm.weight,
                                      eps=self.ffn_norm.eps, lin_b=ff.w3)
        y = decode_layer.linear_fused(g, ff.w2, residual=h)
        return y.view(B, 1, dim)


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
