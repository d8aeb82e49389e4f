"""Dense, pre-allocated KV cache (interface of src/kv_cache.py:4-57).

Layout (must stay bit-identical to the reference):
    k, v : [n_layers, max_batch_size, n_kv_heads, max_seq_len, head_dim]
    element (layer, b, h, pos, d) at flat index
        ((((layer * max_batch + b) * n_kv_heads + h) * max_seq + pos) * head_dim + d)
Each layer's block [max_batch, n_kv_heads, max_seq, head_dim] is contiguous,
so a decode step streams whole 256 B (D=128 bf16) rows of one (b, h) head.
On MI355X the whole cache of the bench configs (a few GB) lives in HBM.

Writes go through the HIP append kernel (``mi_rope_kv_append`` with RoPE
disabled): no host synchronisation, legal under hipGraph capture.
"""
from __future__ import annotations

import torch

from . import _lib
from .config import ModelArgs


class KVCache:
    def __init__(self, args: ModelArgs, dtype: torch.dtype | None = None):
        self.n_layers = args.n_layers
        self.max_batch_size = args.max_batch_size
        self.max_seq_len = args.max_seq_len
        self.n_kv_heads = args.n_kv_heads
        self.head_dim = args.dim // args.n_heads
        self.dtype = dtype if dtype is not None else torch.get_default_dtype()
        shape = (self.n_layers, self.max_batch_size, self.n_kv_heads,
                 self.max_seq_len, self.head_dim)
        # k holds RoPE-applied keys, v the projected values.
        self.k = torch.zeros(shape, device=args.device, dtype=self.dtype)
        self.v = torch.zeros(shape, device=args.device, dtype=self.dtype)

    def reset(self):
        self.k.zero_()
        self.v.zero_()

    def _write(self, layer_idx: int, k_val: torch.Tensor, v_val: torch.Tensor,
               start_pos: int, positions: torch.Tensor | None) -> None:
        B, H, S, D = k_val.shape
        if v_val.shape != k_val.shape:
            raise ValueError(f"k and v shapes must match, got {tuple(k_val.shape)} and {tuple(v_val.shape)}")
        if B > self.max_batch_size or H != self.n_kv_heads or D != self.head_dim:
            raise ValueError(f"k/v shape {tuple(k_val.shape)} does not fit the cache "
                             f"[{self.max_batch_size}, {self.n_kv_heads}, *, {self.head_dim}]")
        ck = self.k[layer_idx, :B]
        cv = self.v[layer_idx, :B]
        k_val = k_val.to(self.dtype)
        v_val = v_val.to(self.dtype)
        lib = _lib.load()
        code = _lib.dtype_code(self.dtype)
        st = lib.mi_rope_kv_append(
            k_val.data_ptr(), v_val.data_ptr(), None, None,
            ck.data_ptr(), cv.data_ptr(), int(start_pos), _lib.ptr(positions), 0,
            B, H, S, D, self.max_seq_len,
            *k_val.stride(), *v_val.stride(), *ck.stride(), *cv.stride(),
            0, 0, 0, 0, 0, code, code, _lib.stream_of(ck))
        _lib.check(st, "KVCache write")

    def update(self, layer_idx, start_pos, k_val, v_val):
        """Write k/v [B, Hkv, S, D] at positions start_pos..start_pos+S-1 and
        return the [:, :, :start_pos+S] views (src/kv_cache.py:23-35)."""
        batch_size = k_val.size(0)
        seq_len = k_val.size(2)
        end_pos = start_pos + seq_len
        self._write(layer_idx, k_val, v_val, start_pos, None)
        return (self.k[layer_idx, :batch_size, :, :end_pos],
                self.v[layer_idx, :batch_size, :, :end_pos])

    def update_positions(self, layer_idx, positions, k_val, v_val, return_full: bool = False):
        """Scatter k/v token s to slot positions[s] (src/kv_cache.py:37-57).

        With return_full=False the visible length is max(positions)+1, which
        needs a host read (as in the reference); return_full=True is graph-safe.
        """
        if positions.dim() != 1:
            raise ValueError(f"positions must be a 1D tensor, got shape={tuple(positions.shape)}")
        batch_size = k_val.size(0)
        if positions.size(0) != k_val.size(2):
            raise ValueError(
                f"positions length mismatch: positions={positions.size(0)} vs seq_len={k_val.size(2)}")
        pos = positions.to(device=self.k.device, dtype=torch.int64)
        self._write(layer_idx, k_val, v_val, 0, pos)
        layer_k = self.k[layer_idx, :batch_size]
        layer_v = self.v[layer_idx, :batch_size]
        if return_full:
            return layer_k, layer_v
        end_pos = int(pos.max().item()) + 1
        return layer_k[:, :, :end_pos], layer_v[:, :, :end_pos]
