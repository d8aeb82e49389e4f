"""Decode-step output projection: final RMSNorm + lm_head (+ greedy argmax).

The reference computes a decode step's logits as ``self.output(self.norm(h))``
(src/model.py:137, :183) — an RMSNorm launch and a bf16 GEMM through the
vendor library — and greedy sampling as ``torch.argmax(logit, dim=-1)``
(src/sampler.py:30) followed by ``next_token.item()`` on the host
(main.py:260).  ``lm_head`` runs the same math as one HIP launch
(mi_lm_head: the normalised rows staged once per workgroup, the weight matrix
streamed once), and with ``greedy=True`` also returns the argmax token of
every row as a device int64 tensor from a second, tiny launch — no host sync,
so a whole greedy token loop can stay inside a captured hipGraph.

Results: logits are rounded to the activation dtype after fp32 accumulation
(as the reference's Linear output is); the argmax is exactly
``torch.argmax(logits, -1)`` of these logits (first index among equal maxima).
"""
from __future__ import annotations

import torch

from . import _lib


def supported(M: int, K: int, weight: torch.Tensor, norm_weight=None) -> bool:
    """Whether ``lm_head`` takes [M, K] rows through `weight` [N, K]."""
    dt = weight.dtype
    if dt not in (torch.bfloat16, torch.float16):
        return False
    if not (1 <= M <= 16 and K % 512 == 0 and 512 <= K <= 4096):
        return False
    if not (weight.is_cuda and weight.dim() == 2 and weight.shape[1] == K
            and weight.stride(1) == 1 and weight.data_ptr() % 16 == 0
            and (weight.stride(0) * 2) % 16 == 0):
        return False
    if norm_weight is not None and (norm_weight.dtype != dt or not norm_weight.is_contiguous()
                                    or norm_weight.data_ptr() % 16 != 0):
        return False
    return True


def lm_head(h: torch.Tensor, weight: torch.Tensor, norm_weight: torch.Tensor | None = None,
            eps: float = 1e-6, *, greedy: bool = False):
    """logits = (rmsnorm(h) if norm_weight is given else h) @ weight.T.

    h: [..., K] with at most 16 rows in total (decode); weight: [N, K].
    Returns logits [..., N] (h's dtype), and with ``greedy=True`` the pair
    (logits, tokens) where tokens [...] int64 is the per-row argmax.
    """
    K = h.shape[-1]
    lead = h.shape[:-1]
    x = h.reshape(-1, K)
    M = x.shape[0]
    N = weight.shape[0]
    if x.dtype != weight.dtype:
        raise TypeError(f"lm_head: activation dtype {x.dtype} != weight dtype {weight.dtype}")
    _lib.require_device(x, "lm_head")
    if not supported(M, K, weight, norm_weight):
        raise NotImplementedError(f"lm_head: no kernel for M={M} K={K} {weight.dtype}")
    if x.stride(1) != 1 or x.data_ptr() % 16 != 0 or (x.stride(0) * 2) % 16 != 0:
        x = x.contiguous()
    y = torch.empty((M, N), device=x.device, dtype=x.dtype)
    lib = _lib.load()
    tokens = part_v = part_i = None
    n_parts = 0
    if greedy:
        n_parts = int(lib.mi_lm_head_partials(M, N))
        tokens = torch.empty((M,), device=x.device, dtype=torch.int64)
        part_v = torch.empty((M, n_parts), device=x.device, dtype=torch.float32)
        part_i = torch.empty((M, n_parts), device=x.device, dtype=torch.int32)
    st = lib.mi_lm_head(
        x.data_ptr(), x.stride(0), _lib.ptr(norm_weight), float(eps),
        weight.data_ptr(), weight.stride(0), y.data_ptr(), y.stride(0),
        _lib.ptr(tokens), _lib.ptr(part_v), _lib.ptr(part_i), n_parts,
        M, N, K, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(st, "lm_head")
    logits = y.reshape(*lead, N)
    if greedy:
        return logits, tokens.reshape(lead)
    return logits
