"""Seeded random-shape sweeps of the HIP kernels against the CPU oracle.

The fixed-shape parity tests pin the benchmark configurations and the
reference's own test shapes; these sweeps draw ragged sizes, head groupings,
strides, split counts and dtypes from a seeded generator (one case per seed,
reproducible by its id) to catch tiling and tail mistakes the chosen shapes
miss.  Bars as in the fixed tests: bf16 outputs 2e-2 and fp16 5e-3 max-abs
(attention) or relative to the output scale (W8A16), fp32 LSE 1e-3.
"""
import random

import pytest
import torch

from helpers import max_abs, randn
from oracle import attention as ora
from oracle import quant as oq

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3}


@pytest.mark.parametrize("seed", range(32))
def test_prefill_random_shapes(dev, seed):
    """Random shapes, head dims 16-256, q as a view of [B,S,H,D] memory or
    contiguous, and (half the cases) q's RoPE fused into the kernel with the
    table sliced at a random start row or indexed by random positions."""
    from src.flash_attn import flash_attention
    from src.rope import build_rope_cos_sin, precompute_freqs_cis
    from oracle import rope as orope
    rng = random.Random(1000 + seed)
    B = rng.randint(1, 3)
    Hkv = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 3, 4, 6, 8])
    D = rng.choice([16, 32, 64, 128, 256])
    S = rng.randint(1, 640)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    bshd = rng.random() < 0.5
    rope = rng.choice([None, "rows", "positions"])
    Hq = Hkv * G
    if bshd:
        q = randn((B, S, Hq, D), seed, dtype, dev).transpose(1, 2)
    else:
        q = randn((B, Hq, S, D), seed, dtype, dev)
    k = randn((B, Hkv, S, D), seed + 1, dtype, dev)
    v = randn((B, Hkv, S, D), seed + 2, dtype, dev)
    kw, qref = {}, q.cpu()
    if rope is not None:
        T = S + 64
        cos, sin = build_rope_cos_sin(precompute_freqs_cis(D, T, theta=500000.0), dtype, dev)
        if rope == "rows":
            r0 = rng.randint(0, 64)
            c_, s_ = cos[r0:r0 + S], sin[r0:r0 + S]
            kw = dict(rope_cos=c_, rope_sin=s_)
            qref = orope.rotate(qref, c_.cpu(), s_.cpu())
        else:
            pos = torch.randperm(T, generator=torch.Generator().manual_seed(seed))[:S]
            kw = dict(rope_cos=cos, rope_sin=sin, rope_positions=pos.to(dev))
            qref = orope.rotate(qref, cos.cpu()[pos], sin.cpu()[pos])
    out, lse = flash_attention(q, k, v, return_lse=True, **kw)
    ref, ref_lse = ora.prefill(qref, k, v)
    case = (B, Hkv, G, D, S, dtype, bshd, rope)
    assert max_abs(out, ref) < TOL[dtype], case
    assert max_abs(lse, ref_lse) < 1e-3, case


@pytest.mark.parametrize("seed", range(40))
def test_decode_random_shapes(dev, seed):
    from src.flash_decode import flash_decode
    rng = random.Random(2000 + seed)
    B = rng.randint(1, 6)
    Hkv = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 3, 4, 6])
    D = rng.choice([64, 128])
    L = rng.randint(1, 2500)
    T = L + rng.choice([0, 16, 100])               # cache capacity beyond the view
    dtype = rng.choice([torch.bfloat16, torch.float16])
    splits = rng.choice([None, 1, 2, 5, 16, 33])
    use_lens = rng.random() < 0.6
    q = randn((B, Hkv * G, 1, D), seed, dtype, dev)
    k = randn((B, Hkv, T, D), seed + 1, dtype, dev)[:, :, :L]
    v = randn((B, Hkv, T, D), seed + 2, dtype, dev)[:, :, :L]
    seq_lens = None
    if use_lens:
        lens = [rng.randint(0, L) for _ in range(B)]
        seq_lens = torch.tensor(lens, dtype=torch.int64, device=dev)
    out, lse = flash_decode(q, k, v, num_splits=splits, seq_lens=seq_lens, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v, seq_lens=seq_lens)
    case = (B, Hkv, G, D, L, T, dtype, splits, None if seq_lens is None else seq_lens.tolist())
    assert max_abs(out, ref) < TOL[dtype], case
    finite = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse.cpu()), finite), case     # empty rows: -inf
    if finite.any():
        assert max_abs(lse.cpu()[finite], ref_lse[finite]) < 1e-3, case


@pytest.mark.parametrize("seed", range(40))
def test_w8a16_random_shapes(dev, seed):
    """W8A16Linear-level dispatch (GEMV, GEMV slices, GEMM, split-K) and the
    GEMM entry with a forced split count, on strided activation rows."""
    from src.quant_linear import W8A16Linear, w8a16_gemm_mfma
    from src.quant_utils import quantize_weight_symmetric_per_channel
    rng = random.Random(3000 + seed)
    M = rng.choice([rng.randint(1, 40), rng.randint(1, 700)])
    N = rng.randint(1, 1600)
    K = 64 * rng.randint(1, 32)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    sdtype = rng.choice([dtype, torch.float32])
    pad = 8 * rng.randint(0, 4)
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn(N, K, generator=g).to(dtype).to(dev)
    q, s = quantize_weight_symmetric_per_channel(w)
    s = s.to(sdtype)
    x = torch.randn(M, K + pad, generator=g).to(dtype).to(dev)[:, :K]
    ref = oq.w8a16(x, q, s)
    scale = float(ref.float().abs().max()) + 1e-6
    case = (M, N, K, dtype, sdtype, pad)
    layer = W8A16Linear(K, N).to(dev)
    layer.weight.data, layer.scales.data = q, s
    assert max_abs(layer(x), ref) < 2e-2 * scale, case
    nk = K // 64
    splits = rng.choice([1] + [v for v in (2, 3, 8) if v <= nk])
    assert max_abs(w8a16_gemm_mfma(x, q, s, splits=splits), ref) < 2e-2 * scale, case + (splits,)
