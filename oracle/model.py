"""CPU composition of one Llama-3 decode step, in the order of the reference's
Attention/TransformerBlock/Llama3 forward (src/model.py:39-185,
src/model_quantized.py:42-190).  TEST INFRASTRUCTURE ONLY.

Arithmetic is fp32; values are rounded to the activation dtype at the points
where the engine stores them (after each projection, norm, RoPE, attention and
residual add), so differences against the GPU come from summation order only.
The composition is pinned against transformers' LlamaForCausalLM run on the
same checkpoint in fp32 (tests/test_oracle_model.py).
"""
from __future__ import annotations

import math

import torch

from . import attention as ora
from . import quant as oq
from . import rope as orope


def _lin(x, layer_mod, dt):
    """nn.Linear (bf16 weight) or W8A16Linear (int8 + scales)."""
    if hasattr(layer_mod, "scales"):
        return oq.w8a16(x, layer_mod.weight, layer_mod.scales)
    w = layer_mod.weight.detach().to("cpu", torch.float32)
    return (x.to(torch.float32) @ w.t()).to(dt)


@torch.no_grad()
def decode_step(model, tokens: torch.Tensor, pos: int, cache_k: torch.Tensor,
                cache_v: torch.Tensor, eps: float):
    """One decode token per row at position `pos` for every row.

    model: the engine's module tree (weights are read, never its kernels);
    tokens [B, 1]; cache_k/cache_v CPU copies [L, MB, Hkv, T, D] holding slots
    < pos (updated in place with slot pos).  Returns logits [B, 1, vocab] fp32.
    """
    args = model.args
    dt = model.tok_embeddings.weight.dtype
    B = tokens.shape[0]
    H, Hkv = args.n_heads, args.n_kv_heads
    D = args.dim // H
    h = model.tok_embeddings.weight.detach().cpu()[tokens.cpu()].to(dt)  # [B,1,dim]
    fc = orope.freqs_cis(D, args.max_seq_len, args.rope_theta, args.rope_scaling)
    cos, sin = orope.cos_sin(fc[pos:pos + 1], dt)
    for li, layer in enumerate(model.layers):
        att = layer.attention
        x = oq.rmsnorm(h, layer.attention_norm.weight, eps)
        xq = _lin(x, att.wq, dt).view(B, 1, H, D).transpose(1, 2)
        xk = _lin(x, att.wk, dt).view(B, 1, Hkv, D).transpose(1, 2)
        xv = _lin(x, att.wv, dt).view(B, 1, Hkv, D).transpose(1, 2)
        xq = orope.rotate(xq, cos, sin)
        cache_k[li, :B, :, pos] = orope.rotate(xk, cos, sin)[:, :, 0].to(cache_k.dtype)
        cache_v[li, :B, :, pos] = xv[:, :, 0].to(cache_v.dtype)
        out, _ = ora.decode(xq, cache_k[li, :B, :, :pos + 1], cache_v[li, :B, :, :pos + 1])
        out = out.to(dt).transpose(1, 2).reshape(B, 1, H * D)
        h = (h.float() + _lin(out, att.wo, dt).float()).to(dt)
        ff = layer.feed_forward
        x = oq.rmsnorm(h, layer.ffn_norm.weight, eps)
        a = _lin(x, ff.w1, dt).float()
        g = (a * torch.sigmoid(a)).to(dt).float() * _lin(x, ff.w3, dt).float()
        h = (h.float() + _lin(g.to(dt), ff.w2, dt).float()).to(dt)
    x = oq.rmsnorm(h, model.norm.weight, eps)
    w = model.output.weight.detach().to("cpu", torch.float32)
    return x.float() @ w.t()
