"""Build libmiattn.so: every HIP source in csrc/ compiled for gfx950 and linked.

Usage: python build_lib.py [--report]     (--report prints per-kernel VGPR/LDS use)

The library is built in-tree (next to this file) so it travels with the repo
snapshot to the GPU box; it is never pip-installed.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIB = HERE / "libmiattn.so"
INCLUDE = HERE.parent / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 VALU ops are disabled for all device code.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# Extra flags per source.  prefill: scores are never NaN for finite inputs, and
# without NaN semantics the row max compiles to plain v_max/v_max3 instead of
# canonicalise+max pairs (the -inf causal mask is unaffected); the ILP-first
# machine scheduler orders its softmax/MFMA slots ~1.5-2 % faster than the
# default occupancy-first one (same 2 waves per SIMD, no spills).
PER_FILE = {"prefill.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def _compile(src: Path, report: bool) -> tuple[Path, str]:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *COMMON, *PER_FILE.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if report:
        cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the device-only target feature; drop that
    # harmless warning so real diagnostics stay visible.
    log = "\n".join(
        ln for ln in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in ln and "--hip-link" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, log


def build(report: bool = False, jobs: int | None = None) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, log in ex.map(lambda s: _compile(s, report), srcs):
            objs.append(obj)
            if log.strip():
                print(log, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--report", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args()
    lib = build(report=args.report, jobs=args.jobs)
    print(f"built {lib}")


if __name__ == "__main__":
    main()
