"""CPU: pin the attention oracle against independent formulations.

Each check is chosen so a plausible oracle mistake fails it: a wrong GQA map
(h % G instead of h // G), a missing or doubled scale, an off-by-one causal
mask, a wrong LSE base, a wrong empty-row or combine rule.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora


def _r(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g)


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2), (6, 2)])
def test_prefill_matches_sdpa(Hq, Hkv):
    q, k, v = _r((2, Hq, 33, 64), 0), _r((2, Hkv, 33, 64), 1), _r((2, Hkv, 33, 64), 2)
    out, _ = ora.prefill(q, k, v)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)


def test_prefill_brute_force_loops():
    B, Hq, Hkv, S, D = 1, 4, 2, 6, 8
    q, k, v = _r((B, Hq, S, D), 3), _r((B, Hkv, S, D), 4), _r((B, Hkv, S, D), 5)
    out, lse = ora.prefill(q, k, v)
    for h in range(Hq):
        kh = h // (Hq // Hkv)
        for i in range(S):
            s = [sum(float(q[0, h, i, d]) * float(k[0, kh, j, d]) for d in range(D)) / math.sqrt(D)
                 for j in range(i + 1)]
            mx = max(s)
            z = sum(math.exp(x - mx) for x in s)
            assert abs(float(lse[0, h, i]) - (mx + math.log(z))) < 1e-5
            for d in range(D):
                o = sum(math.exp(s[j] - mx) * float(v[0, kh, j, d]) for j in range(i + 1)) / z
                assert abs(float(out[0, h, i, d]) - o) < 1e-5


def test_prefill_special_cases():
    q, k, v = _r((1, 4, 16, 32), 6), _r((1, 2, 16, 32), 7), _r((1, 2, 16, 32), 8)
    out, lse = ora.prefill(q, k, v)
    # row 0 attends only key 0
    assert torch.allclose(out[0, :, 0], v[0, [0, 0, 1, 1], 0], atol=1e-6)
    s00 = (q[0, :, 0] * k[0, [0, 0, 1, 1], 0]).sum(-1) / math.sqrt(32)
    assert torch.allclose(lse[0, :, 0], s00, atol=1e-5)
    # constant keys -> uniform weights -> prefix mean of V
    kc = torch.ones_like(k)
    out_c, lse_c = ora.prefill(q, kc, v)
    prefix = v.cumsum(2) / torch.arange(1, 17).view(1, 1, 16, 1)
    assert torch.allclose(out_c, prefix.repeat_interleave(2, dim=1), atol=1e-5)
    # extra cache rows beyond S are ignored (keys are bounded by S)
    k_long = torch.cat([k, _r((1, 2, 5, 32), 9)], dim=2)
    v_long = torch.cat([v, _r((1, 2, 5, 32), 10)], dim=2)
    assert torch.equal(ora.prefill(q, k_long, v_long)[0], out)


def test_decode_matches_sdpa_with_mask():
    B, Hq, Hkv, L, D = 3, 6, 2, 40, 16
    q, k, v = _r((B, Hq, 1, D), 11), _r((B, Hkv, L, D), 12), _r((B, Hkv, L, D), 13)
    mask = torch.rand(B, L, generator=torch.Generator().manual_seed(1)) < 0.5
    out, lse = ora.decode(q, k, v, mask=mask)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask[:, None, None, :], enable_gqa=True)
    assert torch.allclose(out, ref, atol=1e-5)
    scores = (q.repeat(1, 1, 1, 1) @ k.repeat_interleave(3, 1).transpose(-1, -2))[:, :, 0] / 4.0
    ref_lse = torch.logsumexp(scores.masked_fill(~mask[:, None], float("-inf")), -1)
    assert torch.allclose(lse, ref_lse, atol=1e-5)


def test_decode_closed_forms():
    q, k, v = _r((2, 4, 1, 8), 14), _r((2, 2, 1, 8), 15), _r((2, 2, 1, 8), 16)
    out, lse = ora.decode(q, k, v)
    assert torch.allclose(out[:, :, 0], v[:, [0, 0, 1, 1], 0])
    k5, v5 = _r((2, 2, 5, 8), 17), _r((2, 2, 5, 8), 18)
    mask = torch.zeros(2, 5, dtype=torch.bool)
    mask[0, 2] = True
    out, lse = ora.decode(q, k5, v5, mask=mask)
    assert torch.all(out[1] == 0) and torch.all(torch.isneginf(lse[1]))
    assert torch.allclose(out[0, :, 0], v5[0, [0, 0, 1, 1], 2])
    out_n, _ = ora.decode(q, k5, v5, mask=mask, empty="nan")
    assert torch.all(torch.isnan(out_n[1]))
    # seq_lens == prefix mask; all-ones mask == no mask
    lens = torch.tensor([3, 5])
    a, _ = ora.decode(q, k5, v5, seq_lens=lens)
    b, _ = ora.decode(q, k5, v5, mask=torch.arange(5)[None] < lens[:, None])
    assert torch.equal(a, b)
    c, _ = ora.decode(q, k5, v5, mask=torch.ones(5, dtype=torch.bool))
    d, _ = ora.decode(q, k5, v5)
    assert torch.equal(c, d)


@pytest.mark.parametrize("split_len", [1, 7, 64, 256, 1000])
def test_split_combine_invariance(split_len):
    B, Hq, Hkv, L, D = 2, 6, 2, 300, 16
    q, k, v = _r((B, Hq, 1, D), 20), _r((B, Hkv, L, D), 21), _r((B, Hkv, L, D), 22)
    mask = torch.rand(B, L, generator=torch.Generator().manual_seed(2)) < 0.3
    mask[1, :] = False  # one empty row
    m, l, acc = ora.split_partials(q, k, v, split_len, mask=mask)
    out, lse = ora.combine(m, l, acc)
    ref, ref_lse = ora.decode(q, k, v, mask=mask)
    assert torch.allclose(out, ref, atol=1e-5)
    assert torch.allclose(lse[0], ref_lse[0], atol=1e-5)
    assert torch.all(out[1] == 0) and torch.all(torch.isneginf(lse[1]))
    # empty splits publish l == 0
    assert bool(((l == 0) | (l >= 1.0)).all())
