"""CPU: pin the quantiser / W8A16 / RMSNorm oracles with hand-built cases and
integer-exact arithmetic (independent of the formulas they check)."""
import numpy as np
import torch

from oracle import quant as oq


def test_bf16_rounding_helper_against_torch_cast():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(10000, generator=g) * 100
    ref = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(oq._round_f32_to(x.numpy(), "bfloat16"), ref)
    assert np.array_equal(oq._round_f32_to(x.numpy(), "float16"), x.half().float().numpy())


def test_quantiser_hand_built_rows():
    w = np.zeros((5, 8), np.float32)
    w[1, 3] = -2.0                       # single element -> -127
    w[2] = [0.5, -1.0, 1.5, 2.0, -2.5, 3.0, -3.5, 4.0]
    w[3, 0] = 1e-20                      # below the 1e-12 clamp
    w[4] = np.linspace(-1, 1, 8)
    q, s = oq.quantize_per_channel(w, "float32")
    assert np.all(q[0] == 0) and s[0, 0] == np.float32(1e-12) / np.float32(127)
    assert q[1, 3] == -127 and np.count_nonzero(q[1]) == 1
    assert q[2, 7] == 127
    assert q[3, 0] == 0  # 1e-20 / (1e-12/127) rounds to 0
    assert np.all(np.abs(q) <= 127)


def test_quantiser_ties_round_half_even():
    # scale = 127/127 = 1 exactly: w = k + 0.5 must round to the even neighbour
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]], np.float32)
    q, s = oq.quantize_per_channel(w, "float32")
    assert s[0, 0] == 1.0
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -2, 4]]


def test_quantiser_bf16_scale_rounded_before_use():
    # amax/127 is not representable in bf16; q uses the rounded scale
    w = np.array([[1.0, 0.3, -0.7]], np.float32)
    q, s = oq.quantize_per_channel(w, "bfloat16")
    exact = np.float32(1.0) / np.float32(127.0)
    assert s[0, 0] != exact and abs(s[0, 0] - exact) < exact * 2 ** -8
    assert q[0, 0] == np.rint(np.float32(1.0) / s[0, 0])
    # abs-max maps to +-127 (or 126 at an exact tie), never -128
    rng = np.random.default_rng(0)
    ww = oq._round_f32_to(rng.standard_normal((64, 256)).astype(np.float32), "bfloat16")
    qq, _ = oq.quantize_per_channel(ww, "bfloat16")
    amax_q = np.abs(qq).max(axis=1)
    assert np.all((amax_q == 127) | (amax_q == 126)) and qq.min() >= -127


def test_w8a16_oracle_integer_exact():
    g = torch.Generator().manual_seed(1)
    x = torch.randint(-3, 4, (3, 64), generator=g).to(torch.bfloat16)
    q = torch.randint(-128, 128, (5, 64), generator=g).to(torch.int8)
    s = torch.tensor([1.0, 0.5, 2.0, 0.25, 4.0]).to(torch.bfloat16).view(5, 1)
    y = oq.w8a16(x, q, s).float()
    for m in range(3):
        for n in range(5):
            acc = sum(int(x[m, k]) * int(q[n, k]) for k in range(64))
            expect = torch.tensor(acc * float(s[n, 0]), dtype=torch.float32).to(torch.bfloat16).float()
            assert y[m, n] == expect


def test_rmsnorm_oracle_constant_rows():
    x = torch.full((2, 16), 3.0)
    x[1] = -0.5
    w = torch.arange(16, dtype=torch.float32)
    y = oq.rmsnorm(x, w, 1e-5)
    for r, c in ((0, 3.0), (1, -0.5)):
        expect = np.sign(c) * w.numpy() / np.sqrt(1 + 1e-5 / c ** 2)
        assert np.allclose(y[r].numpy(), expect, rtol=1e-6)
