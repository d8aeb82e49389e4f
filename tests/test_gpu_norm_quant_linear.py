"""GPU parity: quantiser (bit-exact), W8A16 GEMV, RMSNorm vs the CPU oracle.

W8A16 cases follow the reference's own unit test (tests/quant_unit.py:80-149):
shapes (M,K,N), weight distributions normal/uniform/extreme, 3-D input, fp16,
non-contiguous input; the reference tolerance there is 1.5 max-abs
(tests/quant_unit.py:61), here 2e-2 relative to the output scale.
"""
import numpy as np
import pytest
import torch

from helpers import max_abs
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _weights(N, K, dtype, dist, seed=42):
    g = torch.Generator("cpu").manual_seed(seed)
    if dist == "normal":
        w = torch.randn(N, K, generator=g)
    elif dist == "uniform":
        w = (torch.rand(N, K, generator=g) - 0.5) * 2.0
    else:  # extreme: small values plus a few large outliers
        w = torch.randn(N, K, generator=g) * 1e-2
        idx = torch.randint(0, N * K, (min(10, N * K),), generator=g)
        w.view(-1)[idx] = torch.tensor([10.0, -10.0, 5.0, -5.0, 8.0, -8.0, 3.0, -3.0, 12.0, -12.0])[: idx.numel()]
    return w.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dist", ["normal", "uniform", "extreme"])
def test_quantiser_bit_exact(dev, dtype, dist):
    from src.quant_utils import quantize_weight_symmetric_per_channel
    w = _weights(384, 1000, dtype, dist)
    w[5] = 0  # all-zero row
    q, s = quantize_weight_symmetric_per_channel(w.to(dev))
    assert q.dtype == torch.int8 and s.dtype == dtype and s.shape == (384, 1)
    name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[dtype]
    rq, rs = oq.quantize_per_channel(w.float().numpy(), name)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.float().cpu().numpy(), rs)


def _check_linear(dev, M, K, N, dtype, dist="normal", x_nc=False, seed=42):
    from src.quant_linear import W8A16Linear
    from src.quant_utils import quantize_weight_symmetric_per_channel
    w = _weights(N, K, dtype, dist, seed).to(dev)
    q, s = quantize_weight_symmetric_per_channel(w)
    layer = W8A16Linear(K, N).to(dev)
    layer.weight.data = q
    layer.scales.data = s.to(dtype)
    g = torch.Generator("cpu").manual_seed(seed + 1)
    if x_nc:
        big = torch.randn(K, M + 1, generator=g).to(dtype).to(dev)
        x = big[:, :-1].t()
        assert not x.is_contiguous()
    else:
        x = torch.randn(M, K, generator=g).to(dtype).to(dev)
    y = layer(x)
    ref = oq.w8a16(x, q, s.to(dtype))
    scale = float(ref.float().abs().max()) + 1e-6
    return max_abs(y, ref) / scale


@pytest.mark.parametrize("M,K,N", [(1, 256, 256), (1, 2048, 2048), (1, 2048, 8192),
                                   (1, 8192, 2048), (8, 2048, 2048), (33, 2048, 2048),
                                   (65, 512, 1024), (3, 80, 100)])
def test_w8a16_reference_shapes(dev, M, K, N):
    assert _check_linear(dev, M, K, N, torch.bfloat16) < 2e-2


@pytest.mark.parametrize("dist", ["normal", "uniform", "extreme"])
def test_w8a16_distributions_and_noncontiguous(dev, dist):
    assert _check_linear(dev, 1, 2048, 2048, torch.bfloat16, dist) < 2e-2
    assert _check_linear(dev, 4, 2048, 2048, torch.bfloat16, dist, x_nc=True) < 2e-2


def test_w8a16_fp16_and_3d_input(dev):
    from src.quant_linear import W8A16Linear
    from src.quant_utils import quantize_weight_symmetric_per_channel
    assert _check_linear(dev, 4, 1024, 1024, torch.float16) < 5e-3
    B, S, K, N = 2, 3, 512, 1024
    w = _weights(N, K, torch.bfloat16, "normal", 0).to(dev)
    q, s = quantize_weight_symmetric_per_channel(w)
    layer = W8A16Linear(K, N).to(dev)
    layer.weight.data, layer.scales.data = q, s
    x = torch.randn(B, S, K, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    y = layer(x)
    assert y.shape == (B, S, N)
    ref = oq.w8a16(x.reshape(-1, K), q, s).reshape(B, S, N)
    assert max_abs(y, ref) / float(ref.float().abs().max()) < 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rmsnorm(dev, dtype):
    from src.rms_norm import RMSNorm
    g = torch.Generator("cpu").manual_seed(3)
    x = (torch.randn(8, 1, 2048, generator=g) * 3).to(dtype).to(dev)
    norm = RMSNorm(2048, eps=1e-5).to(dev)
    norm.weight.data = (torch.rand(2048, generator=g) + 0.5).to(dtype).to(dev)
    y = norm(x)
    ref = oq.rmsnorm(x, norm.weight, 1e-5)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert y.dtype == dtype and y.shape == x.shape
    assert max_abs(y, ref) < tol * float(ref.float().abs().max())


@pytest.mark.parametrize("N", [8, 1000, 2048, 2056, 4104, 8192, 8200, 100])
@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                          (torch.bfloat16, torch.float32)])
def test_rmsnorm_row_widths(dev, N, dtype, wdtype):
    """Rows of 1..4 16-byte chunks per thread (N 8..8192 in multiples of 8),
    the element-load kernel past those (N 8200, N 100), weights of x's dtype or
    fp32, and a row start that is only 2-byte aligned (element-load kernel),
    all against the oracle."""
    from src import _lib
    from src.rms_norm import rmsnorm_triton
    g = torch.Generator("cpu").manual_seed(N)
    x = (torch.randn(5, N, generator=g) * 2).to(dtype).to(dev)
    w = (torch.rand(N, generator=g) + 0.5).to(wdtype).to(dev)
    ref = oq.rmsnorm(x, w, 1e-6)
    tol = (2e-2 if dtype == torch.bfloat16 else 2e-3) * float(ref.float().abs().max())
    y = rmsnorm_triton(x, w, 1e-6)
    assert max_abs(y, ref) < tol
    # rows starting one element into the allocation
    buf = torch.empty(5 * N + 1, dtype=dtype, device=dev)
    xs = buf[1:].view(5, N)
    xs.copy_(x)
    ys = torch.empty_like(x)
    st = _lib.load().mi_rmsnorm(xs.data_ptr(), w.data_ptr(), ys.data_ptr(), 5, N, N, N, 1e-6,
                                _lib.dtype_code(dtype), _lib.dtype_code(wdtype), _lib.stream_of(x))
    _lib.check(st, "rmsnorm")
    assert max_abs(ys, ref) < tol


@pytest.mark.parametrize("M,K,N", [(1, 2048, 2048), (1, 8192, 2048), (8, 2048, 2048),
                                   (16, 1024, 512), (24, 2048, 1024), (3, 80, 100)])
def test_w8a16_gemv_kernel_and_small_m_route(dev, M, K, N):
    """The GEMV kernel (mi_w8a16_gemv) on its own, and the small-M route that
    W8A16Linear takes (the decode-step projection kernel in 16-row slices for
    the shapes it serves, else the GEMV kernel), against the oracle."""
    from src.quant_linear import w8a16_gemv_launch, w8a16_rows
    from src.quant_utils import quantize_weight_symmetric_per_channel
    w = _weights(N, K, torch.bfloat16, "normal", 7).to(dev)
    q, s = quantize_weight_symmetric_per_channel(w)
    x = torch.randn(M, K, generator=torch.Generator("cpu").manual_seed(8)).to(torch.bfloat16).to(dev)
    ref = oq.w8a16(x, q, s)
    scale = float(ref.float().abs().max()) + 1e-6
    assert max_abs(w8a16_gemv_launch(x, q, s), ref) / scale < 2e-2
    assert max_abs(w8a16_rows(x, q, s), ref) / scale < 2e-2
