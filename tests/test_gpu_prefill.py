"""GPU parity: causal GQA prefill (HIP MFMA / fp32 VALU) vs the CPU oracle.

bf16 outputs within 2e-2 max-abs of the fp32 oracle on the same bf16 inputs,
fp32 LSE within 1e-3 (north_star); fp16 within 5e-3; fp32 within 1e-3 (the
reference's own test tolerance, src/flash_attn.py:135).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from helpers import max_abs, randn
from oracle import attention as ora
from oracle import rope as orope

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3, torch.float32: 1e-3}


def _fa():
    from src.flash_attn import flash_attention
    return flash_attention


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (24, 8), (8, 8), (16, 8), (8, 1)])
@pytest.mark.parametrize("S", [1, 45, 256, 333])
def test_prefill_matches_oracle(dev, dtype, D, Hq, Hkv, S):
    B = 2
    q = randn((B, Hq, S, D), 1, dtype, dev)
    k = randn((B, Hkv, S, D), 2, dtype, dev)
    v = randn((B, Hkv, S, D), 3, dtype, dev)
    out, lse = _fa()(q, k, v, return_lse=True)
    ref, ref_lse = ora.prefill(q, k, v)
    assert out.dtype == dtype and out.shape == q.shape
    assert max_abs(out, ref) < TOL[dtype]
    assert max_abs(lse, ref_lse) < 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 256])
@pytest.mark.parametrize("Hq,Hkv,S", [(8, 2, 77), (16, 16, 256), (4, 1, 130)])
def test_prefill_other_head_dims(dev, dtype, D, Hq, Hkv, S):
    """head_dim 16, 32 and 256 (the reference kernel takes any power-of-two
    head_dim, src/flash_attn.py:29-32): bf16/fp16 at 32 and 256 on MFMA, 16
    and fp32 on the VALU kernel; with q's RoPE fused and without."""
    from src.rope import apply_rotary
    B = 2
    q = randn((B, S, Hq, D), 80, dtype, dev).transpose(1, 2)
    k = randn((B, Hkv, S, D), 81, dtype, dev)
    v = randn((B, Hkv, S, D), 82, dtype, dev)
    out, lse = _fa()(q, k, v, return_lse=True)
    ref, ref_lse = ora.prefill(q, k, v)
    assert max_abs(out, ref) < TOL[dtype] and max_abs(lse, ref_lse) < 1e-3
    cos, sin = _rope_tables(D, S, dtype, dev)
    fused = _fa()(q, k, v, rope_cos=cos, rope_sin=sin)
    assert torch.equal(fused, _fa()(apply_rotary(q, cos, sin), k, v))


@pytest.mark.parametrize("D", [8, 48, 512])
def test_prefill_head_dim_without_kernel_is_unsupported(dev, D):
    q = randn((1, 4, 16, D), 83, torch.bfloat16, dev)
    with pytest.raises(NotImplementedError, match="head_dim"):
        _fa()(q, q[:, :1], q[:, :1])


def test_reference_selftest_shape(dev):
    """src/flash_attn.py:113-135: B2 H4 S128 D64 fp32 vs SDPA, atol=rtol=1e-3."""
    q = randn((2, 4, 128, 64), 10, torch.float32, dev)
    k = randn((2, 4, 128, 64), 11, torch.float32, dev)
    v = randn((2, 4, 128, 64), 12, torch.float32, dev)
    out = _fa()(q, k, v)
    mask = torch.triu(torch.ones(128, 128) * float("-inf"), diagonal=1)
    ref = F.scaled_dot_product_attention(q.cpu(), k.cpu(), v.cpu(), attn_mask=mask)
    assert torch.allclose(out.cpu(), ref, atol=1e-3, rtol=1e-3)


def test_model_layout_and_cache_views(dev):
    """q is a [B,H,S,D] view of [B,S,H,D] memory; k/v are cache views with a
    larger capacity T (strides (Hkv*T*D, T*D, D, 1)), as in src/model.py:57-79."""
    B, Hq, Hkv, S, T, D = 2, 32, 8, 300, 1024, 64
    q = randn((B, S, Hq, D), 4, torch.bfloat16, dev).transpose(1, 2)
    kc = randn((B, Hkv, T, D), 5, torch.bfloat16, dev)
    vc = randn((B, Hkv, T, D), 6, torch.bfloat16, dev)
    k, v = kc[:, :, :S], vc[:, :, :S]
    out = _fa()(q, k, v)
    assert out.stride() == q.stride()
    ref, _ = ora.prefill(q, k, v)
    assert max_abs(out, ref) < 2e-2
    # keys beyond S are ignored even when the view is longer (src/flash_attn.py:43-55)
    out2 = _fa()(q, kc[:, :, :S + 50], vc[:, :, :S + 50])
    assert torch.equal(out2, out)


def test_config1_rope_prefill_fp32(dev):
    """BASELINE config 1 on the GPU: fp32, B1 S512 32/8 D64, RoPE theta 5e5 on
    Q and K, N(0,1) from seed 0, checked against the CPU oracle."""
    from src.rope import apply_rotary, build_rope_cos_sin, precompute_freqs_cis
    g = torch.Generator("cpu").manual_seed(0)
    q = torch.randn((1, 32, 512, 64), generator=g)
    k = torch.randn((1, 8, 512, 64), generator=g)
    v = torch.randn((1, 8, 512, 64), generator=g)
    fc = precompute_freqs_cis(64, 512, theta=500000.0)
    cos, sin = build_rope_cos_sin(fc, torch.float32, dev)
    qd = apply_rotary(q.to(dev), cos, sin)
    kd = apply_rotary(k.to(dev), cos, sin)
    out, lse = _fa()(qd, kd, v.to(dev), return_lse=True)
    oc, os_ = orope.cos_sin(orope.freqs_cis(64, 512, 500000.0), torch.float32)
    rq, rk = orope.rotate(q, oc, os_), orope.rotate(k, oc, os_)
    assert torch.equal(qd.cpu(), rq) and torch.equal(kd.cpu(), rk)
    ref, ref_lse = ora.prefill(rq, rk, v)
    assert max_abs(out, ref) < 1e-3
    assert max_abs(lse, ref_lse) < 1e-3


def test_config2_full_size(dev):
    """bf16 B4 S2048 32/8 D64, seed 0, Q pre-scaled by 1/8
    and sm_scale=1 (the softmax scale folded into Q; exact for D=64)."""
    g = torch.Generator("cpu").manual_seed(0)
    q = (torch.randn((4, 32, 2048, 64), generator=g) / 8.0).to(torch.bfloat16)
    k = torch.randn((4, 8, 2048, 64), generator=g).to(torch.bfloat16)
    v = torch.randn((4, 8, 2048, 64), generator=g).to(torch.bfloat16)
    out, lse = _fa()(q.to(dev), k.to(dev), v.to(dev), return_lse=True, sm_scale=1.0)
    out, lse = out.cpu(), lse.cpu()
    for b in range(4):  # oracle one batch at a time to bound host memory
        ref, ref_lse = ora.prefill(q[b:b + 1], k[b:b + 1], v[b:b + 1], sm_scale=1.0)
        assert max_abs(out[b:b + 1], ref) < 2e-2
        assert max_abs(lse[b:b + 1], ref_lse) < 1e-3


def _rope_tables(D, T, dtype, dev):
    from src.rope import build_rope_cos_sin, precompute_freqs_cis
    return build_rope_cos_sin(precompute_freqs_cis(D, T, theta=500000.0), dtype, dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("by_position", [False, True])
def test_fused_q_rope_is_bitwise_apply_rotary_then_attention(dev, dtype, D, by_position):
    """flash_attention(q, k, v, rope_cos=..., rope_sin=...) rotates q inside the
    kernel: the same bits as apply_rotary(q) followed by flash_attention, in the
    model layout (q a view of [B,S,H,D] memory, k/v cache views), and the
    oracle's RoPE + prefill within the usual bars."""
    from src.rope import apply_rotary
    B, Hq, Hkv, S, T = 2, 16, 4, 203, 512
    q = randn((B, S, Hq, D), 40, dtype, dev).transpose(1, 2)
    kc = randn((B, Hkv, T, D), 41, dtype, dev)
    vc = randn((B, Hkv, T, D), 42, dtype, dev)
    k, v = kc[:, :, :S], vc[:, :, :S]
    cos, sin = _rope_tables(D, T, dtype, dev)
    if by_position:   # full tables, token s at position pos[s] (graph-runner style)
        pos = torch.randperm(T, generator=torch.Generator().manual_seed(3))[:S].to(dev)
        c_, s_, kw = cos, sin, dict(positions=pos)
        ref_q = apply_rotary(q, cos, sin, positions=pos)
        fused = _fa()(q, k, v, return_lse=True, rope_cos=cos, rope_sin=sin, rope_positions=pos)
        oc, os_ = cos.cpu()[pos.cpu()], sin.cpu()[pos.cpu()]
    else:             # tables sliced at the start position, row s for token s
        c_, s_ = cos[37:37 + S], sin[37:37 + S]
        ref_q = apply_rotary(q, c_, s_)
        fused = _fa()(q, k, v, return_lse=True, rope_cos=c_, rope_sin=s_)
        oc, os_ = c_.cpu(), s_.cpu()
    sep = _fa()(ref_q, k, v, return_lse=True)
    assert fused[0].stride() == q.stride()
    assert torch.equal(fused[0], sep[0]) and torch.equal(fused[1], sep[1])
    rq = orope.rotate(q.cpu(), oc, os_)
    assert torch.equal(ref_q.cpu(), rq)
    ref, ref_lse = ora.prefill(rq, k, v)
    assert max_abs(fused[0], ref) < TOL[dtype]
    assert max_abs(fused[1], ref_lse) < 1e-3


def test_fused_q_rope_fp32_and_mixed_tables(dev):
    """fp32 q with fp32 tables (rotated in the fp32 kernel's prologue), and
    tables of another dtype than q (apply_rotary first): the same bits as
    apply_rotary by hand, for D 64 and 128."""
    from src.rope import apply_rotary
    for dtype, tdtype, D in ((torch.float32, torch.float32, 64), (torch.float32, torch.float32, 128),
                             (torch.bfloat16, torch.float32, 64)):
        q = randn((1, 70, 8, D), 50, dtype, dev).transpose(1, 2)
        k = randn((1, 2, 70, D), 51, dtype, dev)
        v = randn((1, 2, 70, D), 52, dtype, dev)
        cos, sin = _rope_tables(D, 70, tdtype, dev)
        a = _fa()(q, k, v, rope_cos=cos, rope_sin=sin)
        b = _fa()(apply_rotary(q, cos, sin), k, v)
        assert torch.equal(a, b)
    with pytest.raises(ValueError, match="rows"):
        _fa()(q, k, v, rope_cos=cos[:10], rope_sin=sin[:10])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_epilogue_store_paths_agree(dev, D, dtype):
    """The MFMA kernels (D 32 / 128 / 256 and the D 64 pipelined one) write
    16-byte-aligned output rows through an LDS-staged whole-row epilogue and
    other rows with 8-byte stores: an output buffer offset by 8 bytes (rows 8-
    but not 16-byte aligned) takes the second path and must hold the same
    bits."""
    from src import _lib
    B, Hq, Hkv, S = 2, 8, 2, 333
    q = randn((B, Hq, S, D), 11, dtype, dev)
    k = randn((B, Hkv, S, D), 12, dtype, dev)
    v = randn((B, Hkv, S, D), 13, dtype, dev)
    out, lse = _fa()(q, k, v, return_lse=True)
    buf = torch.full((B * Hq * S * D + 8,), 5.0, device=dev, dtype=dtype)
    o = buf[4:4 + B * Hq * S * D].view(B, Hq, S, D)
    assert o.data_ptr() % 16 == 8
    lse2 = torch.empty_like(lse)
    lib = _lib.load()
    st = lib.mi_attn_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             lse2.data_ptr(), B, Hq, Hkv, S, S, D,
                             *q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *o.stride()[:3],
                             1.0 / D ** 0.5, _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(st, "mi_attn_prefill")
    torch.cuda.synchronize()
    assert torch.equal(o, out)
    assert torch.equal(lse2, lse)
    assert torch.all(buf[:4] == 5.0) and torch.all(buf[4 + B * Hq * S * D:] == 5.0)
