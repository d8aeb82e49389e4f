"""Shared pytest setup.

`-m "not gpu"` runs on any CPU host (oracle pinning, argument checks, C-ABI
exports); `-m gpu` tests call the HIP kernels through the C ABI on an MI355X
and compare them with the CPU oracle on the same seeded inputs.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "llm-infer-engine_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and libmiattn.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")
