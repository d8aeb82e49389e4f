"""GPU parity of the W8A16 prefill GEMM (mi_w8a16_gemm) against the CPU oracle.

Shapes: the reference unit test's multi-row cases (tests/quant_unit.py:82-90,
33 and 65 rows), the Llama-3.2-1B projection shapes at prefill sizes, and
ragged M / N that leave partial 128 x 256 tiles.  Bars:
  * one-hot activation rows select single weight columns, so every output is
    one exact product q * s rounded once: bit-exact against the CPU rounding
    of the same fp32 product (pins row/column/k indexing, the LDS swizzles,
    the k permutation, the int8 widening and the scale index exactly);
  * random inputs: within 2e-2 of the output scale of the fp32 oracle
    (oracle.quant.w8a16, the reference test's reference), and within 1e-2 of
    the GEMV kernel's result on the same rows (two fp32 summation orders).
"""
import pytest
import torch

from helpers import max_abs
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _quantised(N, K, dtype, dev, seed):
    from src.quant_utils import quantize_weight_symmetric_per_channel
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn(N, K, generator=g).to(dtype).to(dev)
    return quantize_weight_symmetric_per_channel(w)


def _x(M, K, dtype, dev, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(M, K, generator=g).to(dtype).to(dev)


def _rel(a, b):
    return max_abs(a, b) / (float(b.float().abs().max()) + 1e-6)


@pytest.mark.parametrize("M,K,N", [(33, 2048, 2048), (65, 512, 1024), (9, 256, 256), (1, 256, 256),
                                   (128, 512, 256), (300, 1024, 1000), (257, 640, 1003)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_matches_oracle_and_gemv(dev, M, K, N, dtype):
    from src.quant_linear import w8a16_gemm_mfma, w8a16_gemv_launch
    q, s = _quantised(N, K, dtype, dev, 1)
    x = _x(M, K, dtype, dev, 2)
    y = w8a16_gemm_mfma(x, q, s)
    assert y.shape == (M, N) and y.dtype == dtype
    ref = oq.w8a16(x, q, s)
    assert _rel(y, ref) < 2e-2
    assert _rel(y, w8a16_gemv_launch(x, q, s)) < 1e-2


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 2048), (512, 2048, 8192), (1024, 8192, 2048),
                                   (640, 2048, 512), (2048, 2048, 8192), (2000, 512, 8000)])
def test_gemm_llama_projection_shapes(dev, M, K, N):
    from src.quant_linear import w8a16_gemm_mfma
    q, s = _quantised(N, K, torch.bfloat16, dev, 3)
    x = _x(M, K, torch.bfloat16, dev, 4)
    y = w8a16_gemm_mfma(x, q, s)
    assert _rel(y, oq.w8a16(x, q, s)) < 2e-2


@pytest.mark.parametrize("dtype,sdtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                          (torch.float16, torch.float16), (torch.float16, torch.float32)])
@pytest.mark.parametrize("M,K,N", [(300, 256, 1000), (130, 512, 259), (128, 64, 256), (1900, 192, 8101)])
def test_one_hot_rows_bit_exact(dev, dtype, sdtype, M, K, N):
    """Row m of x is v_m * e_{k_m} (v_m a power of two): y[m, n] =
    round(v_m * q[n, k_m] * s[n]) with a single exact fp32 product."""
    from src.quant_linear import w8a16_gemm_mfma
    q, s = _quantised(N, K, dtype, dev, 5)
    s = s.to(sdtype)
    g = torch.Generator("cpu").manual_seed(6)
    k_of = torch.randint(0, K, (M,), generator=g)
    v = torch.pow(2.0, torch.randint(-3, 4, (M,), generator=g).float()) * \
        (torch.randint(0, 2, (M,), generator=g).float() * 2 - 1)
    x = torch.zeros(M, K)
    x[torch.arange(M), k_of] = v
    y = w8a16_gemm_mfma(x.to(dtype).to(dev), q, s)
    qc, sc = q.cpu().float(), s.cpu().float().reshape(-1)
    expect = ((qc[:, k_of].t() * v[:, None]) * sc[None, :]).to(dtype)
    assert torch.equal(y.cpu(), expect)


def test_strided_rows_and_output_padding(dev):
    """x with a row stride wider than K; y written through the C ABI into a
    wider buffer: columns past N keep their sentinel."""
    from src import _lib
    M, K, N = 200, 512, 1001
    q, s = _quantised(N, K, torch.bfloat16, dev, 7)
    base = _x(M, K + 64, torch.bfloat16, dev, 8)
    x = base[:, :K]
    y = torch.full((M, N + 7), 7.0, device=dev, dtype=torch.bfloat16)
    st = _lib.load().mi_w8a16_gemm(
        x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr(), M, N, K,
        x.stride(0), q.stride(0), s.stride(0), y.stride(0),
        _lib.dtype_code(x.dtype), _lib.dtype_code(s.dtype), _lib.stream_of(x))
    _lib.check(st, "w8a16_gemm")
    assert _rel(y[:, :N], oq.w8a16(x, q, s)) < 2e-2
    assert torch.all(y[:, N:] == 7.0)


def test_linear_layer_dispatch(dev):
    """W8A16Linear: M > 8 goes to w8a16_gemm_launch, which takes the GEMM
    kernel from GEMM_MIN_ROWS rows (K % 64 == 0) and the GEMV slices below;
    3-D input keeps its leading shape."""
    from src.quant_linear import W8A16Linear, gemm_supported, GEMM_MIN_ROWS
    K, N = 1024, 768
    q, s = _quantised(N, K, torch.bfloat16, dev, 9)
    layer = W8A16Linear(K, N).to(dev)
    layer.weight.data, layer.scales.data = q, s
    for M in (9, GEMM_MIN_ROWS - 1, GEMM_MIN_ROWS, 4 * 97):
        x = _x(M, K, torch.bfloat16, dev, 10 + M)
        y = layer(x.reshape(1, M, K))
        assert y.shape == (1, M, N)
        assert _rel(y.reshape(M, N), oq.w8a16(x, q, s)) < 2e-2
    assert gemm_supported(GEMM_MIN_ROWS, K) and not gemm_supported(GEMM_MIN_ROWS, 80)


@pytest.mark.parametrize("splits", [2, 3, 7, 16])
@pytest.mark.parametrize("M,K,N,dtype", [(33, 2048, 2048, torch.bfloat16), (65, 512, 1024, torch.float16),
                                         (300, 1024, 1000, torch.bfloat16),
                                         (257, 1152, 1003, torch.bfloat16)])
def test_split_k_matches_oracle_and_unsplit(dev, M, K, N, dtype, splits):
    """Split-K (fp32 partials + ordered reduce) against the oracle and the
    single-pass kernel; 7 splits of 16/18 stages leave uneven split depths."""
    from src.quant_linear import w8a16_gemm_mfma
    if splits > K // 64:
        pytest.skip("more splits than 64-deep stages")
    q, s = _quantised(N, K, dtype, dev, 11)
    x = _x(M, K, dtype, dev, 12)
    y = w8a16_gemm_mfma(x, q, s, splits=splits)
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel(y, oq.w8a16(x, q, s)) < 2e-2
    assert _rel(y, w8a16_gemm_mfma(x, q, s, splits=1)) < 1e-2


@pytest.mark.parametrize("splits", [4, 16])
def test_split_k_one_hot_rows_bit_exact(dev, splits):
    """With one nonzero product per output the split sums are exact, so the
    split path is bit-exact like the single pass."""
    from src.quant_linear import w8a16_gemm_mfma
    M, K, N = 130, 1024, 259
    q, s = _quantised(N, K, torch.bfloat16, dev, 13)
    g = torch.Generator("cpu").manual_seed(14)
    k_of = torch.randint(0, K, (M,), generator=g)
    x = torch.zeros(M, K)
    x[torch.arange(M), k_of] = 1.0
    y = w8a16_gemm_mfma(x.to(torch.bfloat16).to(dev), q, s, splits=splits)
    expect = (q.cpu().float()[:, k_of].t() * s.cpu().float().reshape(-1)[None, :]).to(torch.bfloat16)
    assert torch.equal(y.cpu(), expect)


def test_split_k_default_rule_and_strided_output(dev):
    """The library's split count is used by default for small grids; the
    reduce honours a wider output row stride (columns past N untouched)."""
    from src import _lib
    from src.quant_linear import w8a16_gemm_mfma
    M, K, N = 96, 2048, 1536
    lib = _lib.load()
    S = lib.mi_w8a16_gemm_splits(M, N, K)
    assert S > 1
    q, s = _quantised(N, K, torch.bfloat16, dev, 15)
    x = _x(M, K, torch.bfloat16, dev, 16)
    assert _rel(w8a16_gemm_mfma(x, q, s), oq.w8a16(x, q, s)) < 2e-2
    y = torch.full((M, N + 5), 3.0, device=dev, dtype=torch.bfloat16)
    part = torch.empty(S * M * N, device=dev, dtype=torch.float32)
    st = lib.mi_w8a16_gemm_splitk(x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr(), M, N, K,
                                  x.stride(0), q.stride(0), s.stride(0), y.stride(0),
                                  part.data_ptr(), part.numel(), S, 0, 0, _lib.stream_of(x))
    _lib.check(st, "w8a16_gemm_splitk")
    assert _rel(y[:, :N], oq.w8a16(x, q, s)) < 2e-2
    assert torch.all(y[:, N:] == 3.0)


def test_epilogue_store_paths_agree(dev):
    """16-byte-aligned y rows take the LDS-staged whole-line epilogue, rows
    only 8-byte aligned (row stride 1028) the 8-byte stores: same bits."""
    from src import _lib
    M, K, N = 300, 512, 1024
    q, s = _quantised(N, K, torch.bfloat16, dev, 9)
    x = _x(M, K, torch.bfloat16, dev, 10)
    lib = _lib.load()
    ys = []
    for stride in (N, N + 4):
        y = torch.full((M, stride), 3.0, device=dev, dtype=torch.bfloat16)
        st = lib.mi_w8a16_gemm(x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr(), M, N, K,
                               x.stride(0), q.stride(0), s.stride(0), y.stride(0),
                               _lib.dtype_code(x.dtype), _lib.dtype_code(s.dtype), _lib.stream_of(x))
        _lib.check(st, "w8a16_gemm")
        ys.append(y)
    assert (N + 4) * 2 % 16 == 8
    assert torch.equal(ys[0], ys[1][:, :N])
    assert torch.all(ys[1][:, N:] == 3.0)
    assert _rel(ys[0], oq.w8a16(x, q, s)) < 2e-2


@pytest.mark.parametrize("M,K,Ns,dtype", [(8192, 2048, (2048, 512, 512), torch.bfloat16),
                                          (300, 1024, (1000, 256, 77), torch.float16),
                                          (65, 512, (256,), torch.bfloat16),
                                          (1030, 640, (512, 1003, 256, 2048), torch.bfloat16)])
def test_gemm_multi_is_bitwise_the_separate_gemms(dev, M, K, Ns, dtype):
    """Several matrices of one x in one launch (the q/k/v projections): every
    output bitwise the unsplit single-matrix GEMM, ragged N included."""
    from src.quant_linear import w8a16_gemm_mfma, w8a16_gemm_multi
    mats = [_quantised(N, K, dtype, dev, 20 + i) for i, N in enumerate(Ns)]
    x = _x(M, K, dtype, dev, 30)
    ys = w8a16_gemm_multi(x, mats)
    for (q, s), y, N in zip(mats, ys, Ns):
        assert y.shape == (M, N) and y.dtype == dtype
        assert torch.equal(y, w8a16_gemm_mfma(x, q, s, splits=1))
    q, s = mats[-1]
    assert _rel(ys[-1], oq.w8a16(x, q, s)) < 2e-2


def test_gemm_multi_fp32_scales_and_rejections(dev):
    from src import _lib
    from src.quant_linear import w8a16_gemm_mfma, w8a16_gemm_multi
    M, K = 256, 512
    mats = [_quantised(N, K, torch.bfloat16, dev, 40 + N) for N in (512, 256)]
    mats = [(q, s.float()) for q, s in mats]
    x = _x(M, K, torch.bfloat16, dev, 41)
    for (q, s), y in zip(mats, w8a16_gemm_multi(x, mats)):
        assert torch.equal(y, w8a16_gemm_mfma(x, q, s, splits=1))
    with pytest.raises(ValueError):
        w8a16_gemm_multi(x, mats * 3)
    with pytest.raises(TypeError):
        w8a16_gemm_multi(x, [mats[0], (mats[1][0], mats[1][1].bfloat16())])
    # K not a multiple of 64: refused before any launch
    xb = _x(M, 96, torch.bfloat16, dev, 42)
    qb, sb = _quantised(64, 96, torch.bfloat16, dev, 43)
    with pytest.raises(Exception, match="multiple of 64"):
        w8a16_gemm_multi(xb, [(qb, sb)])
    assert "multiple of 64" in _lib.last_error()


def test_quantized_attention_fuses_qkv_at_prefill_sizes(dev):
    """QuantizedAttention.qkv takes the one-launch path when the tiles fill the
    GPU (bitwise the unsplit GEMMs) and the per-linear path otherwise."""
    from src.config import ModelArgs
    from src.model_quantized import QuantizedAttention
    from src.quant_linear import gemm_multi_worth, w8a16_gemm_mfma
    args = ModelArgs(dim=2048, n_layers=1, n_heads=32, n_kv_heads=8, vocab_size=128,
                     max_batch_size=1, max_seq_len=4096)
    attn = QuantizedAttention(args).to(dev)
    for i, lin in enumerate((attn.wq, attn.wk, attn.wv, attn.wo)):
        q, s = _quantised(lin.out_features, lin.in_features, torch.bfloat16, dev, 50 + i)
        lin.weight.data.copy_(q)
        lin.scales.data.copy_(s.view(-1, 1))
    x = _x(4 * 2048, 2048, torch.bfloat16, dev, 60).view(4, 2048, 2048)
    assert gemm_multi_worth(4 * 2048, 2048, [2048, 512, 512], dev)
    xq, xk, xv = attn.qkv(x)
    for y, lin in zip((xq, xk, xv), (attn.wq, attn.wk, attn.wv)):
        assert y.shape == (4, 2048, lin.out_features)
        assert torch.equal(y.view(-1, lin.out_features),
                           w8a16_gemm_mfma(x.view(-1, 2048), lin.weight, lin.scales, splits=1))
        assert _rel(y, lin(x)) < 1e-2
    small = x[:1, :40]
    assert not gemm_multi_worth(40, 2048, [2048, 512, 512], dev)
    for y, lin in zip(attn.qkv(small), (attn.wq, attn.wk, attn.wv)):
        assert torch.equal(y, lin(small))


@pytest.mark.parametrize("M,K,N,dtype,sdtype", [(8192, 2048, 8192, torch.bfloat16, torch.bfloat16),
                                                (300, 1024, 1000, torch.float16, torch.float16),
                                                (65, 512, 200, torch.bfloat16, torch.float32)])
def test_gemm_swiglu_is_the_unfused_chain(dev, M, K, N, dtype, sdtype):
    """silu(w1(x)) * w3(x) in one launch: the GEMM outputs are the unsplit
    single GEMM's bits, then silu and the product are rounded where separate
    ops round.  The kernel's silu (hardware exp2 and reciprocal) rounds to
    the correctly rounded silu (float64, then the dtype) or to one of its two
    neighbours: every output equals bf16(s * y3) for one of those three s
    (an element-exact statement of "silu within one ulp"), and > 99 % of them
    equal the chain with the correctly rounded silu.  The exception is silu
    below 2^-100 (y1 < about -65): the hardware exp2 and reciprocal flush
    fp32 denormals, so there the output may be 0 where the float64 silu is a
    tiny number -- checked as an absolute difference below 2^-80.  Also
    against the fp32 oracle."""
    from src.quant_linear import w8a16_gemm_mfma, w8a16_gemm_swiglu
    q1, s1 = _quantised(N, K, dtype, dev, 70)
    q3, s3 = _quantised(N, K, dtype, dev, 71)
    s1, s3 = s1.to(sdtype), s3.to(sdtype)
    x = _x(M, K, dtype, dev, 72)
    y = w8a16_gemm_swiglu(x, q1, s1, q3, s3)
    assert y.shape == (M, N) and y.dtype == dtype
    y1 = w8a16_gemm_mfma(x, q1, s1, splits=1).cpu()
    y3 = w8a16_gemm_mfma(x, q3, s3, splits=1).cpu().float()
    y1d = y1.double()
    s_cr = (y1d / (1.0 + torch.exp(-y1d))).to(dtype)           # correctly rounded silu
    bits = s_cr.view(torch.int16)
    yc = y.cpu()
    chain = (s_cr.float() * y3).to(dtype)
    ok = yc == chain
    for step in (-1, 1):                                        # the neighbouring values
        nb = (bits + step).view(dtype)
        ok |= yc == (nb.float() * y3).to(dtype)
    tiny = s_cr.float().abs() < 2.0 ** -100
    ok |= tiny & ((yc.float() - chain.float()).abs() <= 2.0 ** -80)
    assert bool(ok.all()), int((~ok).sum())
    assert (yc == chain)[~tiny].float().mean() > 0.99
    assert _rel(yc, chain) < 1e-2
    ref = torch.nn.functional.silu(oq.w8a16(x, q1, s1).float()) * oq.w8a16(x, q3, s3).float()
    assert _rel(yc, ref) < 3e-2


def test_quantized_feed_forward_fuses_at_prefill_sizes(dev):
    from src.model import FeedForward
    from src.model_quantized import QuantizedFeedForward
    from src.quant_linear import swiglu_worth
    ff = QuantizedFeedForward(2048, 8192).to(dev)
    for i, lin in enumerate((ff.w1, ff.w2, ff.w3)):
        q, s = _quantised(lin.out_features, lin.in_features, torch.bfloat16, dev, 80 + i)
        lin.weight.data.copy_(q)
        lin.scales.data.copy_(s.view(-1, 1))
    x = _x(2 * 1024, 2048, torch.bfloat16, dev, 90).view(2, 1024, 2048)
    assert swiglu_worth(2048, 2048, 8192, dev)
    fused = ff(x)
    chain = FeedForward.forward(ff, x)
    assert fused.shape == chain.shape == (2, 1024, 2048)
    assert _rel(fused, chain) < 1e-2
    small = x[:1, :40]
    assert not swiglu_worth(40, 2048, 8192, dev)
    assert torch.equal(ff(small), FeedForward.forward(ff, small))


@pytest.mark.parametrize("M,K,N,dtype,splits,pad", [(8192, 2048, 2048, torch.bfloat16, 1, 0),
                                                    (300, 1024, 1000, torch.float16, 1, 4),
                                                    (64, 8192, 2048, torch.bfloat16, None, 0),
                                                    (100, 512, 256, torch.bfloat16, 4, 4)])
def test_gemm_residual_is_the_separate_add(dev, M, K, N, dtype, splits, pad):
    """res + w8a16(x) with the add in the epilogue, bitwise the GEMM (same
    split count) followed by a separate add; 16-byte residual rows take the
    whole-line path, padded ones (row stride N + 4) the 8-byte one; split-K
    adds the residual in its reduce launch."""
    from src import _lib
    from src.quant_linear import w8a16_gemm_mfma, w8a16_gemm_residual
    q, s = _quantised(N, K, dtype, dev, 100)
    x = _x(M, K, dtype, dev, 101)
    res = _x(M, N + pad, dtype, dev, 102)[:, :N]
    S = _lib.load().mi_w8a16_gemm_splits(M, N, K) if splits is None else splits
    if splits is None:
        assert S > 1
    y = w8a16_gemm_residual(x, q, s, res, splits=S)
    assert torch.equal(y, res + w8a16_gemm_mfma(x, q, s, splits=S))
    with pytest.raises(ValueError):
        w8a16_gemm_residual(x, q, s, res[:, :-1])
