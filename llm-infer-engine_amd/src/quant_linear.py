"""W8A16 linear layer (interface of src/quant_linear.py).

Int8 weights [N, K] with per-row scales [N, 1]; y = (x.f32 @ q.f32^T) * s in
fp32, stored in x's dtype.  Decode-sized inputs (M <= 8 rows, the reference's
threshold at src/quant_linear.py:273) read every weight byte once for all
rows: through the decode-step projection kernel (mi_w8a16_linear_fused with
the plain store epilogue, every weight load issued before the first MFMA)
when the shape is one it serves, otherwise through the MFMA GEMV kernel
mi_w8a16_gemv (any K, strided x, fp32 scales).  Prefill-sized inputs run the
MFMA GEMM mi_w8a16_gemm (128 x 256 output tiles, int8 weight fragments widened
in registers), with K split across workgroups (mi_w8a16_gemm_splitk) when the
tiles alone cannot occupy the GPU.  Between the two, and for K not a multiple
of 64, the small-M kernels serve the rows in 16-row slices: below
GEMM_MIN_ROWS rows (two slices) the slices are faster.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib

_GEMV_MAX_ROWS = 16
GEMM_MIN_ROWS = 33      # rows from which w8a16_gemm_launch uses the GEMM kernels
_GEMM_K_STEP = 64


def _prep(x, weight, scales):
    assert x.dim() == 2
    assert weight.dim() == 2
    assert weight.dtype == torch.int8
    assert x.is_cuda and weight.is_cuda and scales.is_cuda
    assert x.shape[1] == weight.shape[1]
    N = weight.shape[0]
    if scales.dim() == 2:
        assert scales.shape == (N, 1)
        scales_1d = scales.view(N)
    else:
        assert scales.shape == (N,)
        scales_1d = scales
    w = weight
    if w.stride(1) != 1 or w.stride(0) % 16 != 0 or w.data_ptr() % 16 != 0:
        w = w.contiguous()
    if x.stride(1) == 1 and (x.data_ptr() % 16 != 0 or (x.stride(0) * x.element_size()) % 16 != 0):
        x = x.contiguous()
    return x, w, scales_1d


def _gemv_rows(x, w, s, out):
    M, K = x.shape
    N = w.shape[0]
    st = _lib.load().mi_w8a16_gemv(
        x.data_ptr(), w.data_ptr(), s.data_ptr(), out.data_ptr(), M, N, K,
        x.stride(0), x.stride(1), w.stride(0), s.stride(0), out.stride(0), out.stride(1),
        _lib.dtype_code(x.dtype), _lib.dtype_code(s.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_gemv")


# K values and row count the decode-step projection kernel serves
_FUSED_K = (512, 1024, 1536, 2048, 3072, 4096, 6144, 8192)
_FUSED_MAX_ROWS = 16


def _fused_gemv_ok(x, w, s) -> bool:
    M, K = x.shape
    return (1 <= M <= _FUSED_MAX_ROWS and K in _FUSED_K
            and x.dtype in (torch.bfloat16, torch.float16) and s.dtype == x.dtype
            and s.stride(0) == 1 and w.stride(1) == 1 and w.data_ptr() % 16 == 0
            and w.stride(0) % 16 == 0 and x.stride(1) == 1 and x.data_ptr() % 16 == 0
            and (x.stride(0) * x.element_size()) % 16 == 0
            and ((M - 1) * x.stride(0) + K) * 2 < (1 << 31)
            and (w.shape[0] - 1) * w.stride(0) + K < (1 << 31))


def _fused_rows(x, w, s, out):
    M, K = x.shape
    N = w.shape[0]
    st = _lib.load().mi_w8a16_linear_fused(
        x.data_ptr(), x.stride(0), None, 0.0, w.data_ptr(), s.data_ptr(), w.stride(0),
        None, None, 0, None, 0, out.data_ptr(), out.stride(0), M, N, K,
        0, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_linear_fused")


def w8a16_rows(x, weight, scales):
    """Small-M product (decode batches, and the rows below GEMM_MIN_ROWS): the
    decode-step projection kernel in 16-row slices where it serves the shape,
    else the GEMV kernel (same slices)."""
    xp, w, s = _prep(x, weight, scales)
    M = xp.shape[0]
    if not _fused_gemv_ok(xp[:_FUSED_MAX_ROWS], w, s):
        return w8a16_gemv_launch(x, weight, scales)
    out = torch.empty((M, w.shape[0]), device=xp.device, dtype=xp.dtype)
    for m0 in range(0, M, _FUSED_MAX_ROWS):
        _fused_rows(xp[m0:m0 + _FUSED_MAX_ROWS], w, s, out[m0:m0 + _FUSED_MAX_ROWS])
    return out


def w8a16_gemv_launch(x, weight, scales, *, block_n: int = 32, block_k: int = 256):
    """x [M, K] bf16/fp16, weight [N, K] int8, scales [N, 1] or [N] -> [M, N].
    block_n/block_k are accepted for signature compatibility (tiling is fixed
    by the MFMA kernel)."""
    x, w, s = _prep(x, weight, scales)
    M = x.shape[0]
    out = torch.empty((M, w.shape[0]), device=x.device, dtype=x.dtype)
    for m0 in range(0, M, _GEMV_MAX_ROWS):
        _gemv_rows(x[m0:m0 + _GEMV_MAX_ROWS], w, s, out[m0:m0 + _GEMV_MAX_ROWS])
    return out


def gemm_supported(M: int, K: int) -> bool:
    """Whether w8a16_gemm_launch runs the GEMM kernel for an [M, K] input."""
    return M >= GEMM_MIN_ROWS and K % _GEMM_K_STEP == 0


def w8a16_gemm_mfma(x, weight, scales, *, splits: int | None = None):
    """The GEMM kernels for any M (K % 64 == 0): x [M, K] -> [M, N].

    Grids of 128 x 256 tiles that do not occupy the GPU split K across
    workgroups (fp32 partials in a workspace, then one reduce launch); the
    split count comes from mi_w8a16_gemm_splits unless `splits` is given
    (1 = no split)."""
    x, w, s = _prep(x, weight, scales)
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    N = w.shape[0]
    lib = _lib.load()
    out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    S = lib.mi_w8a16_gemm_splits(M, N, K) if splits is None else int(splits)
    args = (x.data_ptr(), w.data_ptr(), s.data_ptr(), out.data_ptr(), M, N, K,
            x.stride(0), w.stride(0), s.stride(0), out.stride(0))
    codes = (_lib.dtype_code(x.dtype), _lib.dtype_code(s.dtype), _lib.stream_of(x))
    if S > 1:
        part = torch.empty(S * M * N, device=x.device, dtype=torch.float32)
        st = lib.mi_w8a16_gemm_splitk(*args, part.data_ptr(), part.numel(), S, *codes)
        _lib.check(st, "w8a16_gemm_splitk")
    else:
        st = lib.mi_w8a16_gemm(*args, *codes)
        _lib.check(st, "w8a16_gemm")
    return out


_GEMM_TILE_M, _GEMM_TILE_N = 128, 256
_CUS: dict = {}


def _cu_count(device) -> int:
    """Compute units of `device` (looked up once per device)."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def w8a16_gemm_residual(x, weight, scales, res, *, splits: int | None = None):
    """res + w8a16(x, weight, scales) with the add in the GEMM epilogue (the
    same roundings as the separate ops): x [M, K], res [M, N] in x's dtype.
    The split rule is w8a16_gemm_mfma's."""
    x, w, s = _prep(x, weight, scales)
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    N = w.shape[0]
    if res.shape != (M, N) or res.dtype != x.dtype or res.device != x.device:
        raise ValueError(f"residual must be [{M}, {N}] {x.dtype} on {x.device}, "
                         f"got {tuple(res.shape)} {res.dtype}")
    if res.stride(1) != 1:
        res = res.contiguous()
    lib = _lib.load()
    out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    S = lib.mi_w8a16_gemm_splits(M, N, K) if splits is None else int(splits)
    part = torch.empty(S * M * N, device=x.device, dtype=torch.float32) if S > 1 else None
    st = lib.mi_w8a16_gemm_residual(
        x.data_ptr(), w.data_ptr(), s.data_ptr(), res.data_ptr(), out.data_ptr(), M, N, K,
        x.stride(0), w.stride(0), s.stride(0), res.stride(0), out.stride(0),
        _lib.ptr(part), 0 if part is None else part.numel(), S,
        _lib.dtype_code(x.dtype), _lib.dtype_code(s.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_gemm_residual")
    return out


def gemm_multi_worth(M: int, K: int, out_features, device) -> bool:
    """Whether one mi_w8a16_gemm_multi launch should serve several projections
    of the same [M, K] input: the GEMM kernels apply and the 128 x 256 tiles of
    all matrices together give every CU a workgroup (smaller grids are better
    served one matrix at a time with K split across workgroups)."""
    if not gemm_supported(M, K):
        return False
    tiles = -(-M // _GEMM_TILE_M) * sum(-(-n // _GEMM_TILE_N) for n in out_features)
    return tiles >= _cu_count(device)


def w8a16_gemm_multi(x, mats):
    """x [M, K] times each (weight [N_i, K] int8, scales [N_i] or [N_i, 1]) of
    `mats` (1-4 pairs) in one launch -> [y_i [M, N_i]]; each y_i is bitwise
    w8a16_gemm_mfma(x, weight_i, scales_i, splits=1)."""
    import ctypes
    if not 1 <= len(mats) <= 4:
        raise ValueError(f"w8a16_gemm_multi takes 1-4 matrices, got {len(mats)}")
    prepped = [_prep(x, w, s) for w, s in mats]
    x = prepped[0][0]
    if x.stride(1) != 1:
        x = x.contiguous()
    sdt = {s.dtype for _, _, s in prepped}
    if len(sdt) != 1:
        raise TypeError("w8a16_gemm_multi: all scales must share a dtype")
    M, K = x.shape
    outs = [torch.empty((M, w.shape[0]), device=x.device, dtype=x.dtype) for _, w, _ in prepped]
    n = len(prepped)
    P = ctypes.c_void_p * n
    I = ctypes.c_int64 * n
    w_arr = P(*[w.data_ptr() for _, w, _ in prepped])
    s_arr = P(*[s.data_ptr() for _, _, s in prepped])
    y_arr = P(*[y.data_ptr() for y in outs])
    n_arr = I(*[w.shape[0] for _, w, _ in prepped])
    wsn = I(*[w.stride(0) for _, w, _ in prepped])
    ssn = I(*[s.stride(0) for _, _, s in prepped])
    ysm = I(*[y.stride(0) for y in outs])
    lib = _lib.load()
    st = lib.mi_w8a16_gemm_multi(
        x.data_ptr(), M, K, x.stride(0), n,
        ctypes.addressof(w_arr), ctypes.addressof(s_arr), ctypes.addressof(y_arr),
        ctypes.addressof(n_arr), ctypes.addressof(wsn), ctypes.addressof(ssn),
        ctypes.addressof(ysm),
        _lib.dtype_code(x.dtype), _lib.dtype_code(prepped[0][2].dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_gemm_multi")
    return outs


def swiglu_worth(M: int, K: int, N: int, device) -> bool:
    """Whether w8a16_gemm_swiglu should serve a W8A16 feed-forward input of
    [M, K] rows: the GEMM kernels apply and its 128 x 128 tiles of the gated
    product give every CU a workgroup."""
    if not gemm_supported(M, K):
        return False
    tiles = -(-M // _GEMM_TILE_M) * -(-N // (_GEMM_TILE_N // 2))
    return tiles >= _cu_count(device)


def w8a16_gemm_swiglu(x, w1, s1, w3, s3):
    """silu(x w1^T * s1) * (x w3^T * s3) in one launch, x [M, K] -> [M, N],
    rounded where silu(w8a16(x, w1, s1)) * w8a16(x, w3, s3) rounds (silu from
    the hardware exp2 and reciprocal: an element may be one ulp off)."""
    x, w1, s1 = _prep(x, w1, s1)
    _, w3, s3 = _prep(x, w3, s3)
    if x.stride(1) != 1:
        x = x.contiguous()
    if w3.shape != w1.shape:
        raise ValueError(f"w1 and w3 shapes differ: {tuple(w1.shape)} and {tuple(w3.shape)}")
    if s1.dtype != s3.dtype:
        raise TypeError("w8a16_gemm_swiglu: s1 and s3 must share a dtype")
    M, K = x.shape
    N = w1.shape[0]
    out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    st = _lib.load().mi_w8a16_gemm_swiglu(
        x.data_ptr(), w1.data_ptr(), s1.data_ptr(), w3.data_ptr(), s3.data_ptr(), out.data_ptr(),
        M, N, K, x.stride(0), w1.stride(0), s1.stride(0), w3.stride(0), s3.stride(0),
        out.stride(0), _lib.dtype_code(x.dtype), _lib.dtype_code(s1.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_gemm_swiglu")
    return out


def w8a16_gemm_launch(x, weight, scales, *, block_m: int = 64, block_n: int = 64, block_k: int = 128):
    """Same contract as w8a16_gemv_launch for any M (src/quant_linear.py:191-247).
    block_m/block_n/block_k are accepted for signature compatibility (the
    MFMA tiling is fixed)."""
    if gemm_supported(x.shape[0], x.shape[1]):
        return w8a16_gemm_mfma(x, weight, scales)
    return w8a16_rows(x, weight, scales)


class W8A16Linear(nn.Module):
    """Per-channel symmetric int8 weight, bf16/fp16 activation linear layer."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        if bias:
            raise NotImplementedError("W8A16Linear does not support bias yet.")
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=torch.int8),
                                   requires_grad=False)
        self.scales = nn.Parameter(torch.empty(out_features, 1, dtype=torch.bfloat16),
                                   requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, self.in_features)
        if x_2d.shape[0] <= 8:
            out_2d = w8a16_rows(x_2d, self.weight, self.scales)
        else:
            out_2d = w8a16_gemm_launch(x_2d, self.weight, self.scales, block_m=64, block_n=64,
                                       block_k=128)
        return out_2d.reshape(*orig_shape[:-1], self.out_features)
