"""CPU: libmiattn.so loads, exports every function include/miattn.h declares,
the ctypes signatures agree with the header, and the C-side argument checks
reject bad calls before any launch (no GPU needed for that)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "miattn.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int32_t|int64_t|const char\*)\s+(mi_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        decls[m.group(1)] = len(params)
    return decls


def test_header_declares_entry_points():
    decls = _declared()
    for name in ("mi_flash_decode", "mi_decode_split", "mi_decode_combine",
                 "mi_rope", "mi_rope_kv_append", "mi_last_error", "mi_version"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    from src import _lib
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in miattn.h but not exported"


def test_ctypes_signatures_match_header():
    from src import _lib
    decls = _declared()
    assert set(decls) == set(_lib.SIGNATURES), "binding table out of sync with header"
    for name, n in decls.items():
        assert len(_lib.SIGNATURES[name][1]) == n, f"{name}: {n} params in header"


def test_version_and_empty_error():
    from src import _lib
    lib = _lib.load()
    assert lib.mi_version() >= 100


def _decode_call(lib, **over):
    args = dict(q=1 << 20, k=1 << 20, v=1 << 20, mask=None, msb=0, msl=0, sl=None,
                pm=1 << 20, pl=1 << 20, pa=1 << 20, B=1, Hq=8, Hkv=8, L=64, D=128,
                S=2, qs=(1024, 128, 1), ks=(8192, 8192, 128), vs=(8192, 8192, 128),
                scale=0.1, dtype=0)
    args.update(over)
    a = args
    return lib.mi_decode_split(a["q"], a["k"], a["v"], a["mask"], a["msb"], a["msl"], a["sl"],
                               a["pm"], a["pl"], a["pa"], a["B"], a["Hq"], a["Hkv"], a["L"],
                               a["D"], a["S"], *a["qs"], *a["ks"], *a["vs"], a["scale"],
                               a["dtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"q": None}, -1, "null"),
    ({"Hq": 12, "Hkv": 8}, -1, "divisible"),
    ({"D": 257}, -2, "head_dim"),
    ({"D": 0}, -1, "positive"),
    ({"dtype": 7}, -1, "dtype"),
    ({"L": 0}, -1, "positive"),
    ({"k": (1 << 20) + 1}, -1, "element size"),     # bf16 K at an odd byte address
    ({"pm": None}, -1, "partial"),
    ({"S": 100000}, -2, "num_splits"),
])
def test_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _decode_call(lib, **over) == code
    assert msg in _lib.last_error()


@pytest.mark.parametrize("head_dim", [1, 4, 7, 0, -3, 300])
def test_split_rules_at_any_head_dim(head_dim):
    """The split-count helpers and the allocation-free entry point take any
    head_dim without dividing by a zero lane count: head dims below one 16-byte
    chunk (bf16 D < 8) get a valid count, and head dims outside 1..256 are
    refused by the launch, not by a crash."""
    from src import _lib
    lib = _lib.load()
    s = lib.mi_decode_effective_splits(1, 8, 2, 4096, head_dim, 2)
    assert s >= 2
    assert lib.mi_decode_default_splits(1, 8, 2, 4096, head_dim) >= 1
    if 1 <= head_dim <= 256:
        return          # a valid call would launch: not with these stand-in pointers
    st = lib.mi_flash_decode_noalloc(1 << 20, 1 << 20, 1 << 20, None, 0, 0, None, 1 << 20, None,
                                     1, 8, 2, 4096, head_dim, 2, 8, 8, 1,
                                     *([1] * 6), 1, 1, 1, 0.1, 0, 0, None)
    assert st in (-1, -2)
    assert "head_dim" in _lib.last_error() or "positive" in _lib.last_error()


def test_rope_kv_append_rejects_out_of_capacity():
    from src import _lib
    lib = _lib.load()
    st = lib.mi_rope_kv_append(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                               60, None, 64, 1, 8, 10, 64, 64,
                               *([1] * 16), 1, 1, 1, 1, 0, 0, 0, None)
    assert st == -1 and "capacity" in _lib.last_error()


@pytest.mark.parametrize("positions,rows", [(None, 9), (1 << 26, 0)])
def test_rope_table_rows_checked_before_launch(positions, rows):
    """Without positions the tables need seq_len (10) rows; with device
    positions (clamped into the table in the kernel) at least one."""
    from src import _lib
    lib = _lib.load()
    st = lib.mi_rope(1 << 20, 1 << 21, 1 << 22, 1 << 23, positions, rows, 1, 8, 10, 64,
                     *([1] * 16), 0, 0, None)
    assert st == -1 and "rows" in _lib.last_error()
    st = lib.mi_rope_kv_append(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                               0, positions, rows, 1, 8, 10, 64, 64,
                               *([1] * 16), 1, 1, 1, 1, int(positions is not None), 0, 0, None)
    assert st == -1 and "rows" in _lib.last_error()


def _prefill_rope_call(lib, **over):
    a = dict(q=1 << 20, k=1 << 21, v=1 << 22, o=1 << 23, B=1, Hq=8, Hkv=2, S=64, L=64, D=64,
             cos=1 << 24, sin=1 << 25, rows=64, rs=32, pos=None, dtype=0)
    a.update(over)
    D = a["D"]
    return lib.mi_attn_prefill_rope(a["q"], a["k"], a["v"], a["o"], None, a["B"], a["Hq"],
                                    a["Hkv"], a["S"], a["L"], D, a["Hq"] * a["S"] * D,
                                    a["S"] * D, D, a["Hkv"] * a["L"] * D, a["L"] * D, D,
                                    a["Hkv"] * a["L"] * D, a["L"] * D, D,
                                    a["Hq"] * a["S"] * D, a["S"] * D, D, 0.125,
                                    a["cos"], a["sin"], a["rows"], a["rs"], a["pos"],
                                    a["dtype"], None)


# every case is rejected before a launch (the pointers are not device memory)
@pytest.mark.parametrize("over,code,msg", [
    ({"dtype": 5}, -1, "dtype"),
    ({"cos": None}, -1, "null"),
    ({"rows": 0}, -1, "rows"),
    ({"rs": 16}, -1, "head_dim/2"),
    ({"sin": (1 << 25) + 4}, -1, "aligned"),
    ({"rows": 32}, -1, "table rows"),
    ({"D": 96, "rs": 48}, -2, "head_dim"),
    ({"Hq": 6, "Hkv": 4}, -1, "divisible"),
])
def test_prefill_rope_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _prefill_rope_call(lib, **over) == code
    assert msg in _lib.last_error()


def _lm_head_call(lib, **over):
    a = dict(x=1 << 20, x_sm=2048, norm=None, eps=1e-5, w=1 << 21, w_sn=2048, y=1 << 22,
             y_sm=1000, tok=None, pv=None, pi=None, n_parts=0, m=8, n=1000, k=2048, dtype=0)
    a.update(over)
    return lib.mi_lm_head(a["x"], a["x_sm"], a["norm"], a["eps"], a["w"], a["w_sn"], a["y"],
                          a["y_sm"], a["tok"], a["pv"], a["pi"], a["n_parts"], a["m"], a["n"],
                          a["k"], a["dtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"x": None}, -1, "null"),
    ({"m": 0}, -1, "positive"),
    ({"dtype": 2}, -2, "dtype"),
    ({"m": 17}, -2, "unsupported"),
    ({"k": 1000, "x_sm": 1000, "w_sn": 1000}, -2, "unsupported"),
    ({"x": (1 << 20) + 8}, -1, "aligned"),
    ({"w_sn": 2040}, -1, "aligned"),
])
def test_lm_head_c_side_validation(over, code, msg):
    """mi_lm_head rejects bad calls before touching the device."""
    from src import _lib
    lib = _lib.load()
    assert _lm_head_call(lib, **over) == code
    assert msg in _lib.last_error()
    assert lib.mi_lm_head_partials(0, 1000) == 0


def test_lm_head_python_rules_without_gpu():
    import torch
    from src import lm_head as lh
    w = torch.zeros(64, 512, dtype=torch.bfloat16)
    assert not lh.supported(4, 512, w)             # host tensor
    with pytest.raises(TypeError, match="dtype"):
        lh.lm_head(torch.zeros(4, 512, dtype=torch.float16), w)
    with pytest.raises(ValueError, match="CUDA"):
        lh.lm_head(torch.zeros(4, 512, dtype=torch.bfloat16), w)


def _gemm_call(lib, **over):
    a = dict(x=1 << 20, w=1 << 21, s=1 << 22, y=1 << 23, m=300, n=1000, k=2048,
             x_sm=2048, w_sn=2048, s_sn=1, y_sm=1000, dtype=0, sdtype=0)
    a.update(over)
    return lib.mi_w8a16_gemm(a["x"], a["w"], a["s"], a["y"], a["m"], a["n"], a["k"],
                             a["x_sm"], a["w_sn"], a["s_sn"], a["y_sm"], a["dtype"],
                             a["sdtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"w": None}, -1, "null"),
    ({"m": 0}, -1, "positive"),
    ({"k": 1000, "x_sm": 1000, "w_sn": 1008}, -2, "multiple of 64"),
    ({"x_sm": 1024}, -1, "strides"),
    ({"y_sm": 999}, -1, "strides"),
    ({"w_sn": 1 << 24}, -1, "strides"),
    ({"x": (1 << 20) + 8}, -1, "aligned"),
    ({"x_sm": 2052}, -1, "aligned"),
    ({"w_sn": 2056}, -1, "aligned"),
    ({"dtype": 2, "sdtype": 2}, -2, "bf16 or fp16"),
])
def test_w8a16_gemm_c_side_validation(over, code, msg):
    """mi_w8a16_gemm rejects bad calls before touching the device."""
    from src import _lib
    lib = _lib.load()
    assert _gemm_call(lib, **over) == code
    assert msg in _lib.last_error()


def test_w8a16_gemm_dispatch_rule():
    from src.quant_linear import gemm_supported, GEMM_MIN_ROWS
    assert GEMM_MIN_ROWS > 8                       # M <= 8 is the GEMV side (src/quant_linear.py:273)
    assert gemm_supported(GEMM_MIN_ROWS, 2048) and not gemm_supported(GEMM_MIN_ROWS - 1, 2048)
    assert not gemm_supported(4096, 80)            # K % 64 != 0: GEMV slices


def _splitk_call(lib, **over):
    a = dict(x=1 << 20, w=1 << 21, s=1 << 22, y=1 << 23, m=300, n=1000, k=2048,
             x_sm=2048, w_sn=2048, s_sn=1, y_sm=1000, part=1 << 24, part_elems=8 * 300 * 1000,
             splits=8, dtype=0, sdtype=0)
    a.update(over)
    return lib.mi_w8a16_gemm_splitk(a["x"], a["w"], a["s"], a["y"], a["m"], a["n"], a["k"],
                                    a["x_sm"], a["w_sn"], a["s_sn"], a["y_sm"], a["part"],
                                    a["part_elems"], a["splits"], a["dtype"], a["sdtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"splits": 1}, -1, "splits"),
    ({"splits": 33}, -1, "splits"),               # K / 64 = 32 stages
    ({"part": None}, -1, "workspace"),
    ({"part_elems": 8 * 300 * 1000 - 1}, -1, "workspace"),
    ({"k": 1000, "x_sm": 1000, "w_sn": 1008}, -2, "multiple of 64"),
    ({"x": None}, -1, "null"),
    ({"dtype": 2}, -2, "bf16 or fp16"),
])
def test_w8a16_gemm_splitk_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _splitk_call(lib, **over) == code
    assert msg in _lib.last_error()


def test_w8a16_gemm_split_rule():
    """Splits only for grids of fewer 128 x 256 tiles than CUs (256 CUs
    without a device): about one workgroup per CU, each split >= 8 stages,
    <= 8 splits, partials <= 64 MiB, and a count every split owns stages of."""
    from src import _lib
    lib = _lib.load()
    assert lib.mi_w8a16_gemm_splits(8192, 2048, 2048) == 1        # 512 tiles
    assert lib.mi_w8a16_gemm_splits(4096, 2048, 2048) == 1        # 256 tiles: every CU
    assert lib.mi_w8a16_gemm_splits(2048, 2048, 2048) == 2        # 128 tiles: half the CUs
    assert lib.mi_w8a16_gemm_splits(8192, 512, 2048) == 2         # wk / wv at M = 8192
    assert lib.mi_w8a16_gemm_splits(128, 2048, 2048) == 4         # 8 tiles, 32 stages
    assert lib.mi_w8a16_gemm_splits(512, 2048, 8192) == 8         # 32 tiles, 128 stages (K = 8192)
    assert lib.mi_w8a16_gemm_splits(128, 2048, 1024) == 2         # 16 stages -> 8 deep each
    assert lib.mi_w8a16_gemm_splits(128, 2048, 512) == 1          # 8 stages: too shallow
    assert lib.mi_w8a16_gemm_splits(100, 1000, 1000) == 1         # K % 64 != 0
    for m, n, k in [(48, 2048, 2048), (512, 2048, 2048), (700, 512, 8192), (256, 8192, 2048),
                    (130, 3000, 1984), (2048, 2048, 512)]:
        s = lib.mi_w8a16_gemm_splits(m, n, k)
        nk = k // 64
        assert 1 <= s <= 8 and (s == 1 or s * m * n * 4 <= 64 << 20)
        if s > 1:
            per = -(-nk // s)
            assert -(-nk // per) == s and per >= 8


def _fused_call(lib, **over):
    a = dict(x=1 << 20, x_sm=2048, norm_w=None, w_a=1 << 21, s_a=1 << 22, w_sn_a=2048,
             w_b=None, s_b=None, w_sn_b=0, res=None, res_sm=0, y=1 << 23, y_sm=2048,
             M=8, N=2048, K=2048, epi=0, dtype=0)
    a.update(over)
    return lib.mi_w8a16_linear_fused(a["x"], a["x_sm"], a["norm_w"], 1e-5, a["w_a"], a["s_a"],
                                     a["w_sn_a"], a["w_b"], a["s_b"], a["w_sn_b"], a["res"],
                                     a["res_sm"], a["y"], a["y_sm"], a["M"], a["N"], a["K"],
                                     a["epi"], a["dtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"x": None}, -1, "null x"),
    ({"M": 17}, -2, "1 <= M <= 16"),
    ({"K": 2000}, -2, "1 <= M <= 16"),
    ({"x_sm": 2052}, -1, "16-byte aligned"),
    ({"x_sm": 1 << 28}, -2, "x row stride"),              # x spans >= 2 GB
    ({"w_sn_a": 2056}, -2, "16-byte aligned"),
    ({"N": 1 << 20}, -2, "weight matrix out of range"),   # 2^20 rows x 2 KB = 2 GB
    ({"w_sn_a": 1 << 21}, -2, "weight matrix out of range"),
    ({"epi": 1}, -1, "needs res"),
    ({"epi": 2, "w_b": 1 << 24, "s_b": 1 << 25, "w_sn_b": 2048, "N": 1 << 20}, -2,
     "weight matrix out of range"),
    ({"epi": 7}, -1, "unknown epilogue"),
])
def test_w8a16_linear_fused_c_side_validation(over, code, msg):
    """mi_w8a16_linear_fused rejects bad calls (including weight matrices and x
    spans past the 32-bit buffer offsets its loads use) before touching the device."""
    from src import _lib
    lib = _lib.load()
    assert _fused_call(lib, **over) == code
    assert msg in _lib.last_error()


def _multi_call(lib, n_mats=3, **over):
    a = dict(x=1 << 20, m=300, k=2048, x_sm=2048, dtype=0, sdtype=0,
             w=[1 << 21, 1 << 22, 1 << 23], s=[1 << 24, 1 << 25, 1 << 26],
             y=[1 << 27, 1 << 28, 1 << 29], n=[2048, 512, 512], w_sn=[2048] * 3,
             s_sn=[1] * 3, y_sm=[2048, 512, 512])
    a.update(over)
    P, I = ctypes.c_void_p * 4, ctypes.c_int64 * 4
    arr = {key: (P if key in ("w", "s", "y") else I)(*(a[key] + [0] * (4 - len(a[key]))))
           for key in ("w", "s", "y", "n", "w_sn", "s_sn", "y_sm")}
    return lib.mi_w8a16_gemm_multi(a["x"], a["m"], a["k"], a["x_sm"], n_mats,
                                   *[ctypes.addressof(arr[key]) for key in
                                     ("w", "s", "y", "n", "w_sn", "s_sn", "y_sm")],
                                   a["dtype"], a["sdtype"], None)


@pytest.mark.parametrize("n_mats,over,code,msg", [
    (0, {}, -1, "matrices"),
    (5, {}, -1, "matrices"),
    (3, {"w": [1 << 21, 0, 1 << 23]}, -1, "null"),
    (3, {"k": 1000, "x_sm": 1000, "w_sn": [1008] * 3}, -2, "multiple of 64"),
    (3, {"y_sm": [2048, 511, 512]}, -1, "strides"),
    (3, {"dtype": 2}, -2, "bf16 or fp16"),
])
def test_w8a16_gemm_multi_c_side_validation(n_mats, over, code, msg):
    """Every matrix is checked (and the count bounded) before any launch."""
    from src import _lib
    lib = _lib.load()
    assert _multi_call(lib, n_mats, **over) == code
    assert msg in _lib.last_error()


def _swiglu_call(lib, **over):
    a = dict(x=1 << 20, w1=1 << 21, s1=1 << 22, w3=1 << 23, s3=1 << 24, y=1 << 25, m=300,
             n=1000, k=2048, x_sm=2048, w1_sn=2048, s1_sn=1, w3_sn=2048, s3_sn=1, y_sm=1000,
             dtype=0, sdtype=0)
    a.update(over)
    return lib.mi_w8a16_gemm_swiglu(a["x"], a["w1"], a["s1"], a["w3"], a["s3"], a["y"], a["m"],
                                    a["n"], a["k"], a["x_sm"], a["w1_sn"], a["s1_sn"],
                                    a["w3_sn"], a["s3_sn"], a["y_sm"], a["dtype"], a["sdtype"],
                                    None)


@pytest.mark.parametrize("over,code,msg", [
    ({"w3": None}, -1, "null"),
    ({"w3_sn": 2040}, -1, "w3 rows"),
    ({"w3": (1 << 23) + 8}, -1, "w3 rows"),
    ({"k": 1000, "x_sm": 1000, "w1_sn": 1008, "w3_sn": 1008}, -2, "multiple of 64"),
    ({"dtype": 2}, -2, "bf16 or fp16"),
])
def test_w8a16_gemm_swiglu_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _swiglu_call(lib, **over) == code
    assert msg in _lib.last_error()


def _residual_call(lib, **over):
    a = dict(x=1 << 20, w=1 << 21, s=1 << 22, res=1 << 23, y=1 << 24, m=300, n=1000, k=2048,
             x_sm=2048, w_sn=2048, s_sn=1, res_sm=1000, y_sm=1000, part=1 << 25,
             part_elems=8 * 300 * 1000, splits=8, dtype=0, sdtype=0)
    a.update(over)
    return lib.mi_w8a16_gemm_residual(a["x"], a["w"], a["s"], a["res"], a["y"], a["m"], a["n"],
                                      a["k"], a["x_sm"], a["w_sn"], a["s_sn"], a["res_sm"],
                                      a["y_sm"], a["part"], a["part_elems"], a["splits"],
                                      a["dtype"], a["sdtype"], None)


@pytest.mark.parametrize("over,code,msg", [
    ({"res": None}, -1, "residual"),
    ({"res_sm": 999}, -1, "residual"),
    ({"splits": 33}, -1, "splits"),               # K / 64 = 32 stages
    ({"part": None}, -1, "workspace"),
    ({"part_elems": 8 * 300 * 1000 - 1}, -1, "workspace"),
    ({"dtype": 2}, -2, "bf16 or fp16"),
])
def test_w8a16_gemm_residual_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _residual_call(lib, **over) == code
    assert msg in _lib.last_error()
