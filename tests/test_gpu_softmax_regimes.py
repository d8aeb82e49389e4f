"""GPU parity of the online-softmax bookkeeping under extreme score patterns.

Seeded N(0,1) inputs keep every score within a few units of the row maximum,
so the kernels' running-maximum updates (taken lazily, only when a new
maximum exceeds the running one by 2^8), the P·V rescales and the prefill's
max-free fast path with its fallback are exercised only on first tiles.  Here
the scores are built to force each path on every tile: keys whose score grows
along the sequence (every later tile holds a new, much larger maximum),
decays along it (the first tile holds the maximum, later ones underflow to
zero), alternates in sign with a large magnitude, or is random but scaled so
that a row's probability mass sits on a few keys.  Bars as everywhere: bf16
2e-2 / fp16 5e-3 / fp32 1e-3 max-abs on outputs, fp32 LSE within 1e-3,
against the CPU oracle on the same rounded inputs.
"""
import math

import pytest
import torch

from helpers import max_abs, randn
from oracle import attention as ora

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3, torch.float32: 1e-3}
REGIMES = ["growing", "decaying", "alternating", "peaked"]


def _scores_inputs(regime, B, Hq, Hkv, S, L, D, dtype, dev, seed):
    """q [B,Hq,S,D], k/v [B,Hkv,L,D] whose scaled scores q.k/sqrt(D) follow
    the regime: direction 0 of q is sqrt(D), so the scaled score of key j is
    about k[..., j, 0] (plus a small random part from the other directions)."""
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Hq, S, D, generator=g) * 0.05
    k = torch.randn(B, Hkv, L, D, generator=g) * 0.05
    v = torch.randn(B, Hkv, L, D, generator=g)
    j = torch.arange(L, dtype=torch.float32)
    if regime == "peaked":
        q = torch.randn(B, Hq, S, D, generator=g) * 3.0
        k = torch.randn(B, Hkv, L, D, generator=g) * 3.0
    else:
        q[..., 0] = math.sqrt(D)
        if regime == "growing":
            k[..., 0] = 0.75 * j
        elif regime == "decaying":
            k[..., 0] = -0.75 * j
        else:  # alternating, large magnitude
            k[..., 0] = torch.where(j.long() % 2 == 0, 60.0, -60.0) + 0.01 * j
    return q.to(dtype).to(dev), k.to(dtype).to(dev), v.to(dtype).to(dev)


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 64),
                                     (torch.bfloat16, 128), (torch.bfloat16, 32),
                                     (torch.bfloat16, 256), (torch.float32, 64)])
def test_prefill_softmax_regimes(dev, regime, dtype, D):
    from src.flash_attn import flash_attention
    B, Hq, Hkv, S = 2, 8, 2, 333
    q, k, v = _scores_inputs(regime, B, Hq, Hkv, S, S, D, dtype, dev, seed=D + len(regime))
    out, lse = flash_attention(q, k, v, return_lse=True)
    ref, ref_lse = ora.prefill(q, k, v)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert max_abs(out, ref) < TOL[dtype], (regime, dtype, D)
    assert max_abs(lse, ref_lse) < 1e-3, (regime, dtype, D)


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("splits", [1, 4, 16])
def test_decode_softmax_regimes(dev, regime, splits):
    from src.flash_decode import flash_decode
    B, Hq, Hkv, L, D = 3, 8, 2, 1500, 128
    q, k, v = _scores_inputs(regime, B, Hq, Hkv, 1, L, D, torch.bfloat16, dev, seed=7 + splits)
    sl = torch.tensor([1500, 777, 33], dtype=torch.int64, device=dev)
    out, lse = flash_decode(q, k, v, seq_lens=sl, num_splits=splits, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v, seq_lens=sl)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert max_abs(out, ref) < TOL[torch.bfloat16], (regime, splits)
    assert max_abs(lse, ref_lse) < 1e-3, (regime, splits)
