"""hipGraph-captured decode step (interface of src/cuda_graph.py).

``CUDAGraphDecodeRunner(model, model_args, kv_cache, device)`` keeps the
reference's name and ``decode(token_id, current_pos) -> logits`` contract
(src/cuda_graph.py:8-70); on ROCm torch.cuda.CUDAGraph is a hipGraph.  What the
MI355X version changes:
  * batch support: one token per sequence, ``batch_size`` rows (the reference
    captures batch 1 only); all rows share the decode position, as the
    reference's scatter path does (src/rope.py:216);
  * nothing is copied from the host per step except the token ids: position
    and per-row visible lengths are written with device fills, and RoPE rows
    are gathered on the device from the model's resident cos/sin table (the
    reference copies a freqs row from the CPU table every step, :64);
  * attention reads exactly pos+1 keys per row through ``seq_lens`` instead of
    scanning all max_seq_len slots behind a rewritten bool mask (:65-66);
  * ``greedy=True`` also captures the greedy argmax of the logits
    (``decode_greedy`` returns the next tokens as a device tensor), so a
    greedy token loop never waits on the host (main.py:259-260 syncs per token).
All launches inside the graph are the HIP kernels of libmiattn.so plus the
library GEMMs/elementwise ops of the model.

A model whose forward does not take ``seq_lens`` (the reference's own Llama3,
src/model.py:145-154) is captured the reference's way instead: a static
``freqs_cis`` row and a static [1, 1, 1, max_seq_len] bool mask, both rewritten
before each replay (src/cuda_graph.py:19-70); ``greedy`` needs the native form.
"""
from __future__ import annotations

import inspect

import torch
import torch.nn as nn

from .config import ModelArgs
from .kv_cache import KVCache


def _accepts(fn, name: str) -> bool:
    try:
        params = inspect.signature(fn).parameters
    except (TypeError, ValueError):
        return False
    return name in params or any(p.kind == p.VAR_KEYWORD for p in params.values())


class CUDAGraphDecodeRunner:
    def __init__(self, model: nn.Module, model_args: ModelArgs, kv_cache: KVCache, device: str,
                 *, batch_size: int | None = None, greedy: bool = False):
        if not str(device).startswith("cuda"):
            raise ValueError("CUDAGraphDecodeRunner requires CUDA device")
        self.model = model
        self.model_args = model_args
        self.kv_cache = kv_cache
        self.device = device
        self.batch_size = int(batch_size or model_args.max_batch_size)
        if self.batch_size > kv_cache.max_batch_size:
            raise ValueError(f"batch_size {self.batch_size} exceeds the cache's max_batch_size "
                             f"{kv_cache.max_batch_size}")
        self.graph = torch.cuda.CUDAGraph()
        B = self.batch_size
        self.static_input_token = torch.zeros((B, 1), dtype=torch.long, device=device)
        self.static_scatter_positions = torch.zeros((1,), dtype=torch.long, device=device)
        self.static_seq_lens = torch.ones((B,), dtype=torch.long, device=device)
        self.static_logits = None
        self.static_tokens = None
        self.greedy = bool(greedy)
        # native form (seq_lens, device RoPE rows) or the reference's (freqs row + mask)
        self.native = _accepts(model.forward, "seq_lens")
        if not self.native:
            if self.greedy:
                raise ValueError("greedy=True needs a model whose forward takes seq_lens and "
                                 "greedy")
            fc = model.freqs_cis
            self.static_freqs_cis = torch.zeros((1, fc.shape[-1]), dtype=fc.dtype, device=device)
            self.static_decode_mask = torch.zeros((1, 1, 1, model_args.max_seq_len),
                                                  dtype=torch.bool, device=device)
            self.static_decode_mask[..., 0] = True
            self.static_freqs_cis.copy_(fc[:1].to(device))
        self._capture()

    def _forward(self):
        if not self.native:
            return self.model(self.static_input_token, kv_cache=self.kv_cache,
                              freqs_cis=self.static_freqs_cis, use_cuda_graph=True,
                              scatter_positions=self.static_scatter_positions,
                              decode_attn_mask=self.static_decode_mask)
        out = self.model(self.static_input_token, kv_cache=self.kv_cache, use_cuda_graph=True,
                         scatter_positions=self.static_scatter_positions,
                         seq_lens=self.static_seq_lens, greedy=self.greedy)
        if self.greedy:
            logits, self.static_tokens = out
            return logits
        return out

    def _capture(self):
        torch.cuda.nvtx.range_push("CUDAGraphWarmup")
        warmup_stream = torch.cuda.Stream(device=self.device)
        warmup_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(warmup_stream):
            self._forward()
        torch.cuda.current_stream().wait_stream(warmup_stream)
        torch.cuda.nvtx.range_pop()
        torch.cuda.nvtx.range_push("CUDAGraphCapture")
        with torch.cuda.graph(self.graph):
            self.static_logits = self._forward()
        torch.cuda.nvtx.range_pop()

    def set_inputs(self, token_id, current_pos: int) -> None:
        if current_pos >= self.model_args.max_seq_len or current_pos < 0:
            raise ValueError(f"current_pos out of range: {current_pos}")
        if isinstance(token_id, torch.Tensor):
            self.static_input_token.copy_(token_id.reshape(self.batch_size, 1))
        else:
            self.static_input_token.fill_(int(token_id))
        self.static_scatter_positions.fill_(int(current_pos))
        self.static_seq_lens.fill_(int(current_pos) + 1)
        if not self.native:
            p = int(current_pos)
            self.static_freqs_cis.copy_(self.model.freqs_cis[p:p + 1].to(self.device))
            self.static_decode_mask.zero_()
            self.static_decode_mask[..., :p + 1] = True

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.static_logits

    def decode(self, token_id, current_pos: int) -> torch.Tensor:
        torch.cuda.nvtx.range_push("CUDAGraphReplay")
        self.set_inputs(token_id, current_pos)
        self.graph.replay()
        torch.cuda.nvtx.range_pop()
        return self.static_logits

    def decode_greedy(self, token_id, current_pos: int) -> torch.Tensor:
        """One step and its greedy next tokens [B, 1] (device int64, no host
        sync).  Requires the runner to be built with ``greedy=True``; the
        returned tensor can be passed straight back as the next ``token_id``."""
        if not self.greedy:
            raise ValueError("decode_greedy needs CUDAGraphDecodeRunner(..., greedy=True)")
        self.decode(token_id, current_pos)
        return self.static_tokens
