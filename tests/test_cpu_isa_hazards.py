"""The prefill and W8A16 GEMM tile copies are inline-asm LDS DMAs
(global_load_lds_dwordx4).

The compiler's hazard recognizer does not look inside inline asm, so the asm
must carry its own wait states: the base address SGPRs may have been written by
a VALU instruction (v_readlane / v_readfirstlane after an SGPR spill), which
needs 5 wait states before a VMEM instruction reads them, and M0 (the LDS
destination) needs 1 after its SALU write.  Without them the copy can read a
stale base address and fault.  This test compiles each kernel source that
issues them for gfx950 on the CPU and checks that every LDS DMA is preceded by
``s_nop 4``.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "llm-infer-engine_amd"
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(shutil.which(HIPCC) is None and not Path(HIPCC).exists(),
                    reason="hipcc not available")
@pytest.mark.parametrize("source", ["prefill.hip", "w8a16_gemm.hip"])
def test_lds_dma_has_hazard_padding(tmp_path, source):
    import sys
    sys.path.insert(0, str(PKG))
    import build_lib

    out = tmp_path / (source + ".s")
    cmd = [HIPCC, *build_lib.COMMON, *build_lib.PER_FILE.get(source, []),
           "-S", "--cuda-device-only", str(PKG / "csrc" / source), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [ln.strip() for ln in out.read_text().splitlines()]
    dma = [i for i, ln in enumerate(lines) if ln.startswith("global_load_lds")]
    assert dma, f"no LDS DMA found in {source}"
    for i in dma:
        # the instruction right before the DMA (comments and asm markers skipped)
        j = i - 1
        while j >= 0 and (not lines[j] or lines[j].startswith(";")):
            j -= 1
        assert re.fullmatch(r"s_nop\s+4", lines[j]), (
            f"LDS DMA at asm line {i + 1} of {source} is preceded by '{lines[j]}', not 's_nop 4'")
