"""GPU parity: RoPE and the fused K-RoPE + KV append (HIP) vs the CPU oracle.

The rotation is computed in fp32 with separately rounded products and sum and
rounded once, exactly as the oracle does, so RoPE outputs are compared bit for
bit; cache slot placement and the V copy are bit-exact by construction.
"""
import pytest
import torch

from helpers import randn
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _tables(D, T, dtype, dev, scaling=None):
    from src.rope import build_rope_cos_sin, precompute_freqs_cis
    fc = precompute_freqs_cis(D, T, theta=500000.0, rope_scaling=scaling)
    cos, sin = build_rope_cos_sin(fc, dtype, dev)
    return fc, cos, sin


def test_tables_match_oracle_bitwise(dev):
    scaling = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
               "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    for sc in (None, scaling):
        fc, cos, sin = _tables(64, 4096, torch.bfloat16, dev, sc)
        ofc = orope.freqs_cis(64, 4096, 500000.0, sc)
        oc, os_ = orope.cos_sin(ofc, torch.bfloat16)
        assert torch.equal(cos.cpu(), oc) and torch.equal(sin.cpu(), os_)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_apply_rotary_bitwise(dev, dtype, D):
    from src.rope import apply_rotary
    B, S, H = 2, 37, 8
    # model layout: [B,S,H,D] memory viewed as [B,H,S,D]
    x = randn((B, S, H, D), 1, dtype, dev).transpose(1, 2)
    _, cos, sin = _tables(D, 64, dtype, dev)
    out = apply_rotary(x, cos[5:5 + S], sin[5:5 + S])
    assert out.stride() == x.stride()
    ref = orope.rotate(x, cos[5:5 + S], sin[5:5 + S])
    assert torch.equal(out.cpu(), ref)


def test_rotary_position_zero_is_identity(dev):
    from src.rope import apply_rotary
    x = randn((1, 4, 1, 64), 3, torch.bfloat16, dev)
    _, cos, sin = _tables(64, 8, torch.bfloat16, dev)
    assert torch.equal(apply_rotary(x, cos[:1], sin[:1]), x)


def _cache(n_layers, B, H, T, D, dtype, dev):
    from src.config import ModelArgs
    from src.kv_cache import KVCache
    args = ModelArgs(dim=H * 4 * D, n_layers=n_layers, n_heads=H * 4, n_kv_heads=H,
                     max_batch_size=B, max_seq_len=T, device=str(dev))
    return KVCache(args, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_and_cache_update_sequential(dev, dtype):
    from src.rope import rope_and_cache_update
    n_layers, B, H, T, D, S, start = 3, 2, 8, 256, 64, 40, 17
    kv = _cache(n_layers, B, H, T, D, dtype, dev)
    kv.k.copy_(randn(kv.k.shape, 10, dtype, dev))
    kv.v.copy_(randn(kv.v.shape, 11, dtype, dev))
    before_k, before_v = kv.k.cpu().clone(), kv.v.cpu().clone()
    xk = randn((B, S, H, D), 12, dtype, dev).transpose(1, 2)
    xv = randn((B, S, H, D), 13, dtype, dev).transpose(1, 2)
    _, cos, sin = _tables(D, T, dtype, dev)
    ck, cv = rope_and_cache_update(xk, xv, cos[start:start + S], sin[start:start + S], kv, 1,
                                   start_pos=start)
    assert ck.shape == (B, H, start + S, D)
    assert ck.data_ptr() == kv.k[1].data_ptr()
    ref_k, ref_v = orope.rope_kv_append(before_k, before_v, 1, xk, xv,
                                        cos[start:start + S], sin[start:start + S],
                                        start_pos=start)
    assert torch.equal(kv.k.cpu(), ref_k)
    assert torch.equal(kv.v.cpu(), ref_v)


def test_rope_and_cache_update_scatter_and_slot_formula(dev):
    from src.rope import rope_and_cache_update
    n_layers, B, H, T, D = 2, 4, 8, 128, 64
    kv = _cache(n_layers, B, H, T, D, torch.bfloat16, dev)
    positions = torch.tensor([93], dtype=torch.int64, device=dev)
    xk = randn((B, H, 1, D), 20, torch.bfloat16, dev)
    xv = randn((B, H, 1, D), 21, torch.bfloat16, dev)
    _, cos, sin = _tables(D, T, torch.bfloat16, dev)
    ck, cv = rope_and_cache_update(xk, xv, cos[93:94], sin[93:94], kv, 1,
                                   scatter_positions=positions)
    assert ck.shape == (B, H, T, D)
    flat_v = kv.v.reshape(-1).cpu()
    xv_c = xv.cpu()
    for b in range(B):
        for h in range(H):
            base = orope.kv_slot(1, b, h, 93, 0, B, H, T, D)
            assert torch.equal(flat_v[base:base + D], xv_c[b, h, 0])
    # nothing else was written
    nz = (kv.v.cpu() != 0).nonzero()
    assert set(nz[:, 3].tolist()) == {93} and set(nz[:, 0].tolist()) == {1}
    ref_k = orope.rotate(xk, cos[93:94], sin[93:94])
    assert torch.equal(kv.k[1, :, :, 93].cpu(), ref_k[:, :, 0])


def test_kvcache_update_and_update_positions(dev):
    n_layers, B, H, T, D = 2, 2, 4, 64, 32
    kv = _cache(n_layers, B, H, T, D, torch.bfloat16, dev)
    kval = randn((B, H, 5, D), 30, torch.bfloat16, dev)
    vval = randn((B, H, 5, D), 31, torch.bfloat16, dev)
    k_view, v_view = kv.update(0, 3, kval, vval)
    assert k_view.shape == (B, H, 8, D)
    assert torch.equal(kv.k[0, :, :, 3:8], kval) and torch.equal(kv.v[0, :, :, 3:8], vval)
    pos = torch.tensor([40, 2, 60], device=dev)
    k3 = randn((B, H, 3, D), 32, torch.bfloat16, dev)
    v3 = randn((B, H, 3, D), 33, torch.bfloat16, dev)
    k_view, _ = kv.update_positions(1, pos, k3, v3)
    assert k_view.shape == (B, H, 61, D)
    for i, p in enumerate(pos.tolist()):
        assert torch.equal(kv.k[1, :, :, p], k3[:, :, i])
        assert torch.equal(kv.v[1, :, :, p], v3[:, :, i])


@pytest.mark.parametrize("dtype,tdtype", [(torch.bfloat16, torch.float32),
                                          (torch.float16, torch.float16),
                                          (torch.float16, torch.float32)])
def test_apply_rotary_positions_and_mixed_tables_bitwise(dev, dtype, tdtype):
    """Tables by absolute position (device positions), the 16-byte path
    (same-dtype tables) and the per-element path (fp32 tables) alike."""
    from src.rope import apply_rotary
    B, S, H, D, T = 2, 29, 4, 128, 200
    x = randn((B, S, H, D), 60, dtype, dev).transpose(1, 2)
    _, cos, sin = _tables(D, T, tdtype, dev)
    pos = torch.randperm(T, generator=torch.Generator().manual_seed(1))[:S].to(dev)
    out = apply_rotary(x, cos, sin, positions=pos)
    ref = orope.rotate(x, cos.cpu()[pos.cpu()], sin.cpu()[pos.cpu()])
    assert torch.equal(out.cpu(), ref)


def test_rope_and_cache_update_fp16_and_unaligned_fallback(dev):
    """fp16 through the 16-byte path; a head_dim of 40 (not a multiple of 16)
    through the per-element path; both bitwise against the oracle."""
    from src.rope import rope_and_cache_update
    for dtype, D in ((torch.float16, 64), (torch.bfloat16, 40)):
        n_layers, B, H, T, S, start = 2, 2, 4, 96, 33, 9
        kv = _cache(n_layers, B, H, T, D, dtype, dev)
        before_k, before_v = kv.k.cpu().clone(), kv.v.cpu().clone()
        xk = randn((B, S, H, D), 70, dtype, dev).transpose(1, 2)
        xv = randn((B, S, H, D), 71, dtype, dev).transpose(1, 2)
        _, cos, sin = _tables(D, T, dtype, dev)
        rope_and_cache_update(xk, xv, cos[start:start + S], sin[start:start + S], kv, 0,
                              start_pos=start)
        ref_k, ref_v = orope.rope_kv_append(before_k, before_v, 0, xk, xv,
                                            cos[start:start + S], sin[start:start + S],
                                            start_pos=start)
        assert torch.equal(kv.k.cpu(), ref_k) and torch.equal(kv.v.cpu(), ref_v)


@pytest.mark.parametrize("dtype,tdtype", [(torch.bfloat16, torch.bfloat16),
                                          (torch.bfloat16, torch.float32)])
def test_positions_outside_the_table_use_the_nearest_row(dev, dtype, tdtype):
    """Device positions are not checked on the host (that would need a sync):
    a position outside the table's rows reads the nearest row, never past
    the table, for Q RoPE and for the cache append by absolute position."""
    from src.rope import apply_rotary, rope_and_cache_update
    B, H, D, T = 2, 4, 64, 48
    pos = torch.tensor([-5, 0, 47, 48, 1000], dtype=torch.int64, device=dev)
    clamped = pos.clamp(0, T - 1)
    _, cos, sin = _tables(D, T, tdtype, dev)
    x = randn((B, H, pos.numel(), D), 90, dtype, dev)
    out = apply_rotary(x, cos, sin, positions=pos)
    assert torch.equal(out.cpu(), orope.rotate(x, cos.cpu()[clamped.cpu()], sin.cpu()[clamped.cpu()]))
    # cache append: slots 40..55 of a 64-slot cache, table rows 0..47
    kv = _cache(1, B, H, 64, D, dtype, dev)
    slots = torch.arange(40, 56, device=dev)
    xk = randn((B, H, slots.numel(), D), 91, dtype, dev)
    xv = randn((B, H, slots.numel(), D), 92, dtype, dev)
    rope_and_cache_update(xk, xv, cos, sin, kv, 0, scatter_positions=slots, cos_by_position=True)
    rows = slots.clamp(max=T - 1).cpu()
    ref_k = orope.rotate(xk, cos.cpu()[rows], sin.cpu()[rows])
    assert torch.equal(kv.k[0, :, :, 40:56].cpu(), ref_k)
    assert torch.equal(kv.v[0, :, :, 40:56].cpu(), xv.cpu())
