"""CPU: pin the RoPE/KV oracle with float64 maths and invariants, and check the
product package's host-side tables equal the oracle's bit for bit."""
import math

import torch

from oracle import rope as orope

SCALING = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
           "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def test_inv_freq_formula_float64():
    f = orope.inv_freq(64, 500000.0)
    ref = torch.tensor([500000.0 ** (-(2 * i) / 64) for i in range(32)], dtype=torch.float64)
    assert torch.allclose(f.double(), ref, rtol=2e-6)


def test_llama3_scaling_piecewise():
    base = orope.inv_freq(128, 500000.0)
    f = orope.inv_freq(128, 500000.0, SCALING)
    wl = 2 * math.pi / base.double()
    hi_wl, lo_wl = 8192 / 4.0, 8192 / 1.0
    short = wl < hi_wl
    long_ = wl > lo_wl
    assert torch.equal(f[short], base[short])                       # unchanged
    assert torch.allclose(f[long_], base[long_] / 32.0)            # divided by factor
    mid = ~short & ~long_
    assert mid.any()
    sm = (8192 / wl[mid] - 1.0) / (4.0 - 1.0)
    ref = (1 - sm) * base[mid].double() / 32.0 + sm * base[mid].double()
    assert torch.allclose(f[mid].double(), ref, rtol=1e-6)


def test_tables_against_float64_angles():
    fc = orope.freqs_cis(64, 2048, 500000.0)
    c, s = orope.cos_sin(fc, torch.float32)
    f = orope.inv_freq(64, 500000.0).double()
    ang = torch.arange(2048, dtype=torch.float64)[:, None] * f[None]
    # fp32 angle rounding dominates at large positions: |err| <= ulp(angle)
    tol = (ang.abs() * 2 ** -23).clamp(min=1e-7) + 1e-6
    assert bool(((c.double() - ang.cos()).abs() <= tol).all())
    assert bool(((s.double() - ang.sin()).abs() <= tol).all())


def test_rotation_invariants():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 2, 16, 64, generator=g)
    y = torch.randn(1, 2, 16, 64, generator=g)
    c, s = orope.cos_sin(orope.freqs_cis(64, 64, 10000.0), torch.float32)
    # position 0 is the identity
    assert torch.equal(orope.rotate(x[:, :, :1], c[:1], s[:1]), x[:, :, :1])
    # norms preserved
    rx = orope.rotate(x, c[:16], s[:16])
    assert torch.allclose(rx.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)
    # <R(m)x, R(n)y> depends only on m - n
    x0 = x[:, :, :1].expand(1, 2, 16, 64)
    y0 = y[:, :, :1].expand(1, 2, 16, 64)
    a = (orope.rotate(x0, c[3:19], s[3:19]) * orope.rotate(y0, c[0:16], s[0:16])).sum(-1)
    b = (orope.rotate(x0, c[10:26], s[10:26]) * orope.rotate(y0, c[7:23], s[7:23])).sum(-1)
    assert torch.allclose(a, b, atol=1e-4)
    # rotate-half convention: pair (i, i + D/2) rotates by angle pos*f_i
    e = torch.zeros(1, 1, 1, 64)
    e[..., 0] = 1.0
    r = orope.rotate(e, c[5:6], s[5:6])
    assert torch.allclose(r[0, 0, 0, 0], c[5, 0]) and torch.allclose(r[0, 0, 0, 32], s[5, 0])


def test_kv_slot_formula_matches_contiguous_indexing():
    L, MB, H, T, D = 3, 2, 4, 16, 8
    t = torch.arange(L * MB * H * T * D).reshape(L, MB, H, T, D)
    for idx in [(0, 0, 0, 0, 0), (2, 1, 3, 15, 7), (1, 0, 2, 9, 4)]:
        assert orope.kv_slot(*idx, MB, H, T, D) == int(t[idx])


def test_product_tables_equal_oracle():
    from src.rope import build_rope_cos_sin, precompute_freqs_cis
    for sc in (None, SCALING):
        fc = precompute_freqs_cis(64, 1000, 500000.0, sc)
        assert torch.equal(fc, orope.freqs_cis(64, 1000, 500000.0, sc))
        c, s = build_rope_cos_sin(fc, torch.bfloat16, "cpu")
        oc, os_ = orope.cos_sin(fc, torch.bfloat16)
        assert torch.equal(c, oc) and torch.equal(s, os_)
