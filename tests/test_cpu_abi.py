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
    ({"D": 96}, -2, "head_dim"),
    ({"dtype": 7}, -1, "dtype"),
    ({"L": 0}, -1, "positive"),
    ({"k": (1 << 20) + 2}, -1, "aligned"),
    ({"pm": None}, -1, "partial"),
    ({"S": 100000}, -2, "num_splits"),
])
def test_c_side_validation(over, code, msg):
    from src import _lib
    lib = _lib.load()
    assert _decode_call(lib, **over) == code
    assert msg in _lib.last_error()


def test_rope_kv_append_rejects_out_of_capacity():
    from src import _lib
    lib = _lib.load()
    st = lib.mi_rope_kv_append(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                               60, None, 1, 8, 10, 64, 64,
                               *([1] * 16), 1, 1, 1, 1, 0, 0, 0, None)
    assert st == -1 and "capacity" in _lib.last_error()
