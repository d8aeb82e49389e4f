"""RMSNorm (interface of src/rms_norm.py): y = x * rsqrt(mean(x^2) + eps) * w,
computed in fp32 and stored in x's dtype, one HIP launch (mi_rmsnorm).
``rmsnorm_triton`` keeps the reference's function name for import
compatibility; there is no Triton here."""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        torch.cuda.nvtx.range_push("RMSNorm")
        out = rmsnorm_triton(x, self.weight, self.eps)
        torch.cuda.nvtx.range_pop()
        return out


def rmsnorm_triton(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    assert x.is_cuda
    assert weight.is_cuda
    assert x.shape[-1] == weight.numel()
    orig_shape = x.shape
    N = x.shape[-1]
    x_2d = x.contiguous().view(-1, N)
    w = weight.contiguous()
    y = torch.empty_like(x_2d)
    st = _lib.load().mi_rmsnorm(
        x_2d.data_ptr(), w.data_ptr(), y.data_ptr(), x_2d.shape[0], N,
        x_2d.stride(0), y.stride(0), float(eps),
        _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype), _lib.stream_of(x))
    _lib.check(st, "rmsnorm")
    return y.view(orig_shape)


rmsnorm = rmsnorm_triton
