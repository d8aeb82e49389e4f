"""bf16 Llama-3 module tree (interface of src/model.py) on the HIP hot path.

Attention.forward keeps the reference composition (src/model.py:39-90):
QKV projection -> [B,S,H,D] viewed as [B,H,S,D] -> Q RoPE (apply_rotary) ->
fused K RoPE + KV append (rope_and_cache_update) -> flash_attention when S > 1,
flash_decode when S == 1 -> output projection.  Projections are plain library
GEMMs (torch nn.Linear -> hipBLASLt); everything attention-shaped is a HIP
kernel from libmiattn.so.

Extensions (keyword-only, defaults keep the reference behaviour):
  * ``seq_lens`` [B] device int64: per-sequence visible lengths for decode; the
    kernel reads only those keys (graph-safe, no [B, T] mask rewrite).
  * in graph mode (use_cuda_graph=True with scatter_positions and no explicit
    freqs_cis) cos/sin come from the model's device-resident table indexed by
    the device position, so a replay copies nothing from the host.
  * ``greedy=True`` returns (logits, tokens): tokens [B, 1] int64 is the
    argmax of the returned logits, computed on the device.
The final norm and the output projection of up to 16 rows (decode, or the
last position of a prefill) run as one fused launch (src/lm_head.py).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import lm_head
from .flash_attn import flash_attention
from .flash_decode import flash_decode
from .rms_norm import RMSNorm
from .rope import (
    DeviceRopeTable,
    apply_rotary,
    build_rope_cos_sin,
    precompute_freqs_cis,
    rope_and_cache_update,
)


class FeedForward(nn.Module):
    def __init__(self, dim: int, hidden_dim: int, linear=nn.Linear):
        super().__init__()
        self.w1 = linear(dim, hidden_dim, bias=False)
        self.w2 = linear(hidden_dim, dim, bias=False)
        self.w3 = linear(dim, hidden_dim, bias=False)

    def forward(self, x, *, residual=None):
        """w2(silu(w1(x)) * w3(x)) (src/model.py:21-25); with ``residual``
        (keyword-only extension) residual + that, the block's add."""
        torch.cuda.nvtx.range_push("FFN")
        out = self.down(torch.nn.functional.silu(self.w1(x)) * self.w3(x), residual)
        torch.cuda.nvtx.range_pop()
        return out

    def down(self, h, residual=None):
        out = self.w2(h)
        return out if residual is None else residual + out


class Attention(nn.Module):
    def __init__(self, args, linear=nn.Linear):
        super().__init__()
        self.n_heads = args.n_heads
        self.n_kv_heads = args.n_kv_heads
        self.head_dim = args.dim // args.n_heads
        self.wq = linear(args.dim, args.n_heads * self.head_dim, bias=False)
        self.wk = linear(args.dim, args.n_kv_heads * self.head_dim, bias=False)
        self.wv = linear(args.dim, args.n_kv_heads * self.head_dim, bias=False)
        self.wo = linear(args.n_heads * self.head_dim, args.dim, bias=False)

    def qkv(self, x):
        """The three input projections (src/model.py:54)."""
        return self.wq(x), self.wk(x), self.wv(x)

    def out_proj(self, output, residual=None):
        out = self.wo(output)
        return out if residual is None else residual + out

    def forward(self, x, rope_cos, rope_sin, layer_idx=None, start_pos=0, kv_cache=None,
                use_cuda_graph=False, scatter_positions=None, decode_attn_mask=None, *,
                seq_lens=None, rope_by_position=False, residual=None):
        batch_size, query_len, _ = x.shape
        torch.cuda.nvtx.range_push("QKV_proj")
        xq, xk, xv = self.qkv(x)
        torch.cuda.nvtx.range_pop()
        xq = xq.view(batch_size, query_len, self.n_heads, self.head_dim).transpose(1, 2)
        xk = xk.view(batch_size, query_len, self.n_kv_heads, self.head_dim).transpose(1, 2)
        xv = xv.view(batch_size, query_len, self.n_kv_heads, self.head_dim).transpose(1, 2)

        positions = scatter_positions if (use_cuda_graph and scatter_positions is not None) else None
        q_positions = positions if rope_by_position else None
        if query_len == 1:
            torch.cuda.nvtx.range_push("RoPE")
            xq = apply_rotary(xq, rope_cos, rope_sin, positions=q_positions)
            torch.cuda.nvtx.range_pop()
        # (prefill: q's RoPE runs inside the attention kernel, flash_attention below)

        if kv_cache is not None:
            torch.cuda.nvtx.range_push("KV_cache")
            if layer_idx is None:
                raise ValueError("layer_idx is required when using kv_cache")
            xk, xv = rope_and_cache_update(
                xk, xv, rope_cos, rope_sin, kv_cache, layer_idx,
                start_pos=start_pos, scatter_positions=positions,
                cos_by_position=rope_by_position)
            torch.cuda.nvtx.range_pop()

        if query_len > 1:
            torch.cuda.nvtx.range_push("FlashAttn")
            output = flash_attention(xq, xk, xv, rope_cos=rope_cos, rope_sin=rope_sin,
                                     rope_positions=q_positions)
            torch.cuda.nvtx.range_pop()
        else:
            torch.cuda.nvtx.range_push("FlashDecode")
            output = flash_decode(xq, xk, xv, mask=decode_attn_mask, seq_lens=seq_lens)
            torch.cuda.nvtx.range_pop()

        torch.cuda.nvtx.range_push("Output_proj")
        output = output.transpose(1, 2).contiguous().view(batch_size, query_len, -1)
        out = self.out_proj(output, residual)
        torch.cuda.nvtx.range_pop()
        return out


class TransformerBlock(nn.Module):
    #: the block's attention and feed-forward classes (a subclass swaps in
    #: variants with fused kernels; the parameter names stay the same)
    attention_cls = Attention
    feed_forward_cls = FeedForward

    def __init__(self, args, linear=nn.Linear):
        super().__init__()
        self.attention = self.attention_cls(args, linear)
        self.feed_forward = self.feed_forward_cls(args.dim, args.hidden_dim, linear)
        self.attention_norm = RMSNorm(args.dim, eps=args.norm_eps)
        self.ffn_norm = RMSNorm(args.dim, eps=args.norm_eps)

    def forward(self, x, rope_cos, rope_sin, layer_idx=None, start_pos=0, kv_cache=None,
                use_cuda_graph=False, scatter_positions=None, decode_attn_mask=None, **ext):
        torch.cuda.nvtx.range_push(f"Attn_{layer_idx}")
        # x + attention(...) and x + feed_forward(...) (src/model.py:113-127), the
        # adds passed down so a W8A16 projection can fuse them into its epilogue
        x = self.attention(self.attention_norm(x), rope_cos, rope_sin, layer_idx=layer_idx,
                           start_pos=start_pos, kv_cache=kv_cache,
                           use_cuda_graph=use_cuda_graph, scatter_positions=scatter_positions,
                           decode_attn_mask=decode_attn_mask, residual=x, **ext)
        torch.cuda.nvtx.range_pop()
        torch.cuda.nvtx.range_push(f"FFN_{layer_idx}")
        x = self.feed_forward(self.ffn_norm(x), residual=x)
        torch.cuda.nvtx.range_pop()
        return x


class Llama3(nn.Module):
    block_cls = TransformerBlock
    linear_cls = nn.Linear

    def __init__(self, args):
        super().__init__()
        self.args = args
        self.tok_embeddings = nn.Embedding(args.vocab_size, args.dim)
        self.layers = nn.ModuleList([self.block_cls(args, self.linear_cls)
                                     for _ in range(args.n_layers)])
        self.norm = RMSNorm(args.dim, eps=args.norm_eps)
        self.output = nn.Linear(args.dim, args.vocab_size, bias=False)
        self.freqs_cis = precompute_freqs_cis(args.dim // args.n_heads, args.max_seq_len,
                                              theta=args.rope_theta,
                                              rope_scaling=args.rope_scaling)
        self._rope_table: DeviceRopeTable | None = None

    def rope_table(self, dtype, device) -> DeviceRopeTable:
        """Full cos/sin table resident on the device (built once per dtype/device)."""
        t = self._rope_table
        if t is None or t.cos.dtype != dtype or t.cos.device != torch.device(device):
            t = DeviceRopeTable(self.freqs_cis, dtype, device)
            self._rope_table = t
        return t

    def forward(self, tokens, start_pos=0, kv_cache=None, freqs_cis=None, use_cuda_graph=False,
                scatter_positions=None, decode_attn_mask=None, return_all_logits=False, *,
                seq_lens=None, greedy=False):
        torch.cuda.nvtx.range_push("Embed")
        # the same rows as self.tok_embeddings(tokens); the indexing gather loads
        # every element at once (a decode step's 8 rows: 2.2 us in a hipGraph
        # against 4.2 us for the embedding op, which walks the rows in turn)
        h = self.tok_embeddings.weight[tokens]
        torch.cuda.nvtx.range_pop()
        seq_len = tokens.shape[1]
        by_pos = bool(use_cuda_graph and scatter_positions is not None and freqs_cis is None)
        if by_pos:
            table = self.rope_table(h.dtype, h.device)
            rope_cos, rope_sin = table.cos, table.sin
        elif freqs_cis is None:
            table = self.rope_table(h.dtype, h.device)
            rope_cos, rope_sin = table.rows(start_pos, seq_len)
        else:
            rope_cos, rope_sin = build_rope_cos_sin(freqs_cis, dtype=h.dtype, device=h.device)
        torch.cuda.nvtx.range_push("Layers")
        for layer_idx, layer in enumerate(self.layers):
            h = layer(h, rope_cos, rope_sin, layer_idx=layer_idx, start_pos=start_pos,
                      kv_cache=kv_cache, use_cuda_graph=use_cuda_graph,
                      scatter_positions=scatter_positions, decode_attn_mask=decode_attn_mask,
                      seq_lens=seq_lens, rope_by_position=by_pos)
        torch.cuda.nvtx.range_pop()
        torch.cuda.nvtx.range_push("Output")
        if not return_all_logits and seq_len > 1:
            h = h[:, -1:, :]
        rows = h.shape[0] * h.shape[1]
        if h.is_cuda and lm_head.supported(rows, h.shape[-1], self.output.weight, self.norm.weight):
            # final norm + output projection (+ greedy argmax) in one launch
            out = lm_head.lm_head(h, self.output.weight, self.norm.weight, self.norm.eps,
                                  greedy=greedy)
        else:
            out = self.output(self.norm(h))
            if greedy:
                out = (out, torch.argmax(out, dim=-1))
        torch.cuda.nvtx.range_pop()
        return out
