"""ctypes binding of libmiattn.so (the gfx950 HIP kernels behind this package).

There is exactly one compute path: the HIP kernels.  If the shared library is
missing or cannot be loaded, every op raises — there is no CPU or eager-torch
fallback.  Build the library with ``python llm-infer-engine_amd/build_lib.py``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("MIATTN_LIB", _PKG_ROOT / "libmiattn.so"))

MI_DTYPE_BF16 = 0
MI_DTYPE_F16 = 1
MI_DTYPE_F32 = 2
MI_OK = 0
MI_ERR_INVALID = -1
MI_ERR_UNSUPPORTED = -2

_DTYPE_CODES = {
    torch.bfloat16: MI_DTYPE_BF16,
    torch.float16: MI_DTYPE_F16,
    torch.float32: MI_DTYPE_F32,
}

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p

# name -> (restype, [argtypes]).  Must mirror include/miattn.h exactly.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mi_version": (_i32, []),
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_decode_split": (_i32, [
        _ptr, _ptr, _ptr,            # q k v
        _ptr, _i64, _i64,            # mask, mask_sb, mask_sl
        _ptr,                        # seq_lens
        _ptr, _ptr, _ptr,            # part_m part_l part_acc
        _i64, _i64, _i64, _i64, _i64, _i64,   # B Hq Hkv L D splits
        _i64, _i64, _i64,            # q strides
        _i64, _i64, _i64,            # k strides
        _i64, _i64, _i64,            # v strides
        _f32, _i32, _ptr,            # sm_scale dtype stream
    ]),
    "mi_decode_combine": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr,          # part_m part_l part_acc out lse
        _i64, _i64, _i64, _i64,                # B Hq D splits
        _i64, _i64, _i64,                      # o strides
        _i32, _i32, _ptr,                      # empty_nan dtype stream
    ]),
    "mi_flash_decode": (_i32, [
        _ptr, _ptr, _ptr,
        _ptr, _i64, _i64,
        _ptr,
        _ptr, _ptr, _ptr,
        _ptr,                                  # arrive (in-launch combine counters)
        _ptr, _ptr,                            # out lse
        _i64, _i64, _i64, _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,                      # o strides
        _f32, _i32, _i32, _ptr,                # sm_scale empty_nan dtype stream
    ]),
    "mi_flash_decode_noalloc": (_i32, [
        _ptr, _ptr, _ptr,
        _ptr, _i64, _i64,
        _ptr,
        _ptr, _ptr,                            # out lse
        _i64, _i64, _i64, _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,
        _i64, _i64, _i64,                      # o strides
        _f32, _i32, _i32, _ptr,                # sm_scale empty_nan dtype stream
    ]),
    "mi_decode_arrive_counters": (_i32, [_ptr, _ptr]),      # stream, uint64_t** out
    "mi_decode_default_splits": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "mi_decode_effective_splits": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "mi_attn_prefill": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr,          # q k v out lse
        _i64, _i64, _i64, _i64, _i64, _i64,    # B Hq Hkv S L D
        _i64, _i64, _i64,                      # q strides (b, h, s)
        _i64, _i64, _i64,                      # k strides
        _i64, _i64, _i64,                      # v strides
        _i64, _i64, _i64,                      # out strides
        _f32, _i32, _ptr,                      # sm_scale dtype stream
    ]),
    "mi_attn_prefill_rope": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr,          # q k v out lse
        _i64, _i64, _i64, _i64, _i64, _i64,    # B Hq Hkv S L D
        _i64, _i64, _i64,                      # q strides (b, h, s)
        _i64, _i64, _i64,                      # k strides
        _i64, _i64, _i64,                      # v strides
        _i64, _i64, _i64,                      # out strides
        _f32,                                  # sm_scale
        _ptr, _ptr, _i64, _i64, _ptr,          # cos sin table_rows row_stride positions
        _i32, _ptr,                            # dtype stream
    ]),
    "mi_rope": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr,          # x out cos sin positions
        _i64,                                  # table_rows
        _i64, _i64, _i64, _i64,
        _i64, _i64, _i64, _i64,
        _i64, _i64, _i64, _i64,
        _i64, _i64, _i64, _i64,
        _i32, _i32, _ptr,
    ]),
    "mi_rope_kv_append": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,    # xk xv cos sin cache_k cache_v
        _i64, _ptr, _i64,                      # start_pos positions table_rows
        _i64, _i64, _i64, _i64, _i64,          # B Hkv S D capacity
        _i64, _i64, _i64, _i64,                # xk strides
        _i64, _i64, _i64, _i64,                # xv strides
        _i64, _i64, _i64, _i64,                # ck strides
        _i64, _i64, _i64, _i64,                # cv strides
        _i64, _i64, _i64, _i64,                # cos/sin strides
        _i32, _i32, _i32, _ptr,                # cos_by_pos dtype cdtype stream
    ]),
    "mi_rmsnorm": (_i32, [
        _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _ptr,
    ]),
    "mi_quantize_int8": (_i32, [
        _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i32, _ptr,
    ]),
    "mi_w8a16_gemv": (_i32, [
        _ptr, _ptr, _ptr, _ptr,                # x w scales y
        _i64, _i64, _i64,                      # M N K
        _i64, _i64, _i64, _i64, _i64, _i64,    # x_sm x_sk w_sn s_sn y_sm y_sn
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_gemm": (_i32, [
        _ptr, _ptr, _ptr, _ptr,                # x w scales y
        _i64, _i64, _i64,                      # M N K
        _i64, _i64, _i64, _i64,                # x_sm w_sn s_sn y_sm
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_gemm_splits": (_i64, [_i64, _i64, _i64]),
    "mi_w8a16_gemm_splitk": (_i32, [
        _ptr, _ptr, _ptr, _ptr,                # x w scales y
        _i64, _i64, _i64,                      # M N K
        _i64, _i64, _i64, _i64,                # x_sm w_sn s_sn y_sm
        _ptr, _i64, _i64,                      # part part_elems splits
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_gemm_multi": (_i32, [
        _ptr, _i64, _i64, _i64, _i32,          # x M K x_sm n_mats
        _ptr, _ptr, _ptr,                      # w[] scales[] y[] (host arrays)
        _ptr, _ptr, _ptr, _ptr,                # N[] w_sn[] s_sn[] y_sm[]
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_gemm_swiglu": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,    # x w1 s1 w3 s3 y
        _i64, _i64, _i64,                      # M N K
        _i64, _i64, _i64, _i64, _i64, _i64,    # x_sm w1_sn s1_sn w3_sn s3_sn y_sm
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_gemm_residual": (_i32, [
        _ptr, _ptr, _ptr, _ptr, _ptr,          # x w scales res y
        _i64, _i64, _i64,                      # M N K
        _i64, _i64, _i64, _i64, _i64,          # x_sm w_sn s_sn res_sm y_sm
        _ptr, _i64, _i64,                      # part part_elems splits
        _i32, _i32, _ptr,                      # dtype sdtype stream
    ]),
    "mi_w8a16_linear_fused": (_i32, [
        _ptr, _i64, _ptr, _f32,                # x x_sm norm_w eps
        _ptr, _ptr, _i64,                      # w_a s_a w_sn_a
        _ptr, _ptr, _i64,                      # w_b s_b w_sn_b
        _ptr, _i64, _ptr, _i64,                # res res_sm y y_sm
        _i64, _i64, _i64,                      # M N K
        _i32, _i32, _ptr,                      # epilogue dtype stream
    ]),
    "mi_w8a16_qkv_rope_append": (_i32, [
        _ptr, _i64, _ptr, _f32,                # x x_sm norm_w eps
        _ptr, _ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _i64,   # wq sq wk sk wv sv (+ row strides)
        _ptr, _ptr, _i64, _i64, _i64,          # cos sin c_ss rope_row0 rope_rows
        _ptr, _ptr, _ptr, _ptr,                # pos q_out cache_k cache_v
        _i64, _i64, _i64, _i64,                # c_sb c_sh c_st capacity
        _i64, _i64, _i64, _i64, _i64,          # M K n_heads n_kv_heads head_dim
        _i32, _ptr,                            # dtype stream
    ]),
    "mi_lm_head": (_i32, [
        _ptr, _i64, _ptr, _f32,                # x x_sm norm_w eps
        _ptr, _i64, _ptr, _i64,                # w w_sn y y_sm
        _ptr, _ptr, _ptr, _i64,                # argmax_out part_v part_i n_parts
        _i64, _i64, _i64, _i32, _ptr,          # m n k dtype stream
    ]),
    "mi_lm_head_partials": (_i64, [_i64, _i64]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"libmiattn.so not found at {LIB_PATH}; build it with "
                f"`python {_PKG_ROOT / 'build_lib.py'}` (the HIP kernels are the "
                "only implementation of these ops)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def last_error() -> str:
    return load().mi_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the Python exception the reference would raise."""
    if status == MI_OK:
        return
    msg = f"{what}: {last_error()}"
    if status == MI_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status < 0:
        raise ValueError(msg)
    raise RuntimeError(f"{msg} (hipError {status})")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device (graph-capture aware)."""
    return torch.cuda.current_stream(t.device).cuda_stream


_ARRIVE: dict[tuple[int, int], int | None] = {}
ARRIVE_SLAB = 8192   # MI_DECODE_ARRIVE_SLAB


def arrive_counters(t: torch.Tensor, n_groups: int) -> int | None:
    """Device address of the library's zeroed arrival counters for torch's
    current stream on t's device (mi_decode_arrive_counters; the in-launch LSE
    combine of mi_flash_decode), or None when they cannot serve the call (more
    than a slab's worth of groups, or every slab taken by other streams)."""
    if n_groups > ARRIVE_SLAB:
        return None
    stream = stream_of(t)
    key = (t.device.index if t.device.index is not None else torch.cuda.current_device(), stream)
    if key not in _ARRIVE:
        out = ctypes.c_void_p()
        with torch.cuda.device(t.device):
            st = load().mi_decode_arrive_counters(stream, ctypes.byref(out))
        _ARRIVE[key] = out.value if st == MI_OK else None
    return _ARRIVE[key]


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what} requires CUDA tensors")
