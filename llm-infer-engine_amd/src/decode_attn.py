"""Legacy single-pass decode attention (interface of src/decode_attn.py).

The reference keeps a no-split decode kernel with no callers
(src/decode_attn.py:137-166).  Here the same entry point is served by the
split-KV HIP kernels; the only semantic difference of the legacy kernel that is
kept on purpose is its 0/0: a row whose keys are all masked yields NaN
(src/decode_attn.py:70), where flash_decode yields 0.

Mask strides: the reference passes mask.stride(0) as the batch stride for any
rank, which for a 1-D [L] mask walks the mask by batch index (b + j) and reads
past its end for b > 0.  This build treats a 1-D mask as shared by the batch,
the flash_decode rule (src/flash_decode.py:220-223).
Like the reference, only query token 0 is attended; out is empty_like(xq).
"""
from __future__ import annotations

import torch

from . import _lib
from .flash_decode import _mask_strides, _run_decode  # noqa: F401


def decode_attention(xq, xk, xv, mask=None):
    _lib.require_device(xq, "decode_attention")
    if xq.shape[2] != 1:
        xq_first = xq[:, :, :1]
    else:
        xq_first = xq
    out_first = _run_decode(xq_first, xk, xv, mask, None, None, False, True, "decode_attention")
    if xq.shape[2] == 1:
        return out_first
    out = torch.empty_like(xq)
    out[:, :, :1] = out_first
    return out
