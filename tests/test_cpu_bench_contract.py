"""bench.py's contract on a host without a GPU: one GPU only (--gpus N > 1
exits with a message), a clear failure without a device, and the committed
rocprofv3 traffic summaries it reads for `roofline.traffic` parse."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=600, cwd=str(ROOT))


def test_more_than_one_gpu_is_refused():
    p = _run("--gpus", "8")
    assert p.returncode == 2
    assert "one GPU" in p.stderr and p.stdout == ""


def test_no_device_fails_loudly():
    import torch
    if torch.cuda.is_available():
        import pytest
        pytest.skip("a device is present")
    p = _run("--steps", "1", "--warmup", "0")
    assert p.returncode == 1 and "HIP device" in p.stderr and p.stdout == ""


def test_committed_traffic_summaries_parse():
    sys.path.insert(0, str(ROOT))
    import bench
    for summary, key in [("prefill_config2_traffic.md", "hbm_bytes_per_launch"),
                         ("decode_config3_4_traffic.md", "hbm_bytes_per_launch_config3"),
                         ("w8a16_gemm_traffic.md", "hbm_bytes_per_launch_w1")]:
        v = bench._traffic(summary, key)
        assert isinstance(v, int) and v > 10 ** 7, (summary, key, v)
