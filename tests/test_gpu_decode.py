"""GPU parity: split-KV flash decode (HIP) vs the CPU oracle.

Tolerances (north_star): bf16 outputs within 2e-2 max-abs of the fp32 CPU
oracle on the same bf16 inputs, fp32 LSE within 1e-3.  fp16/fp32 outputs use
tighter bounds (5e-3 / 1e-4).
"""
import pytest
import torch

from helpers import max_abs, randn
from oracle import attention as ora

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3, torch.float32: 1e-4}
LSE_TOL = 1e-3


def _fd():
    from src.flash_decode import flash_decode
    return flash_decode


def _inputs(B, Hq, Hkv, L, D, dtype, dev, seed=0, T=None):
    T = T or L
    q = randn((B, Hq, 1, D), seed, dtype, dev)
    k = randn((B, Hkv, T, D), seed + 1, dtype, dev)[:, :, :L]
    v = randn((B, Hkv, T, D), seed + 2, dtype, dev)[:, :, :L]
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(24, 8), (32, 8), (8, 8), (16, 2)])
def test_decode_matches_oracle(dev, dtype, D, Hq, Hkv):
    B, L = 3, 777
    q, k, v = _inputs(B, Hq, Hkv, L, D, dtype, dev)
    out, lse = _fd()(q, k, v, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v)
    assert out.dtype == dtype and out.shape == q.shape
    assert max_abs(out, ref) < TOL[dtype]
    assert max_abs(lse, ref_lse) < LSE_TOL


@pytest.mark.parametrize("dtype,u", [(torch.bfloat16, 2.0 ** -8), (torch.float16, 2.0 ** -11)])
@pytest.mark.parametrize("D,Hq,Hkv,B,L", [(64, 32, 8, 8, 4097), (128, 24, 8, 3, 777)])
@pytest.mark.parametrize("q_scale", [0.1, 1.0, 8.0])
def test_pv_rounding_bound(dev, dtype, u, D, Hq, Hkv, B, L, q_scale):
    """2-byte K/V fold P.V with each p rounded to the storage type (unit
    roundoff u) and the output rounded once more, so against the fp32 oracle
    |out - ref| <= 2u * max|v| for flat (q_scale 0.1) to peaked (8.0) softmax
    rows, with V of unit and of larger (x 16) magnitude."""
    q, k, v = _inputs(B, Hq, Hkv, L, D, dtype, dev, seed=41)
    q = (q.float() * q_scale).to(dtype)
    for vs in (1.0, 16.0):
        vv = (v.float() * vs).to(dtype)
        out = _fd()(q, k, vv)
        ref, _ = ora.decode(q, k, vv)
        bound = 2 * u * float(vv.abs().max()) + 1e-6
        assert max_abs(out, ref) <= bound, (vs, max_abs(out, ref), bound)


@pytest.mark.parametrize("num_splits", [1, 2, 7, 16, 64, 200])
def test_split_count_invariance(dev, num_splits):
    q, k, v = _inputs(2, 24, 8, 3001, 128, torch.bfloat16, dev, seed=5)
    out, lse = _fd()(q, k, v, num_splits=num_splits, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v)
    assert max_abs(out, ref) < 2e-2
    assert max_abs(lse, ref_lse) < LSE_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 256])
def test_decode_other_head_dims(dev, D, dtype):
    """head_dim 16 / 32 / 256 (the reference's decode takes any power of two up
    to 256, src/flash_decode.py:276-277) through the default split count, a
    single split (no combine), 40 splits (the block-per-row combine), per-
    sequence lengths and a mask."""
    q, k, v = _inputs(2, 6, 2, 515, D, dtype, dev, seed=9)
    sl = torch.tensor([515, 77], dtype=torch.int64, device=dev)
    mask = (torch.rand(2, 515, generator=torch.Generator().manual_seed(2)) < 0.5).to(dev)
    for kw, ref_kw in (({}, {}), ({"num_splits": 1}, {}), ({"num_splits": 40}, {}),
                       ({"seq_lens": sl}, {"seq_lens": sl}), ({"mask": mask}, {"mask": mask})):
        out, lse = _fd()(q, k, v, return_lse=True, **kw)
        ref, ref_lse = ora.decode(q, k, v, **ref_kw)
        assert max_abs(out, ref) < TOL[dtype], (D, dtype, kw.keys())
        assert max_abs(lse, ref_lse) < LSE_TOL, (D, dtype, kw.keys())


@pytest.mark.parametrize("shape", ["1d", "2d", "4d", "4d_b1"])
def test_mask_shapes(dev, shape):
    B, Hq, Hkv, L, D = 4, 24, 8, 1200, 128
    q, k, v = _inputs(B, Hq, Hkv, L, D, torch.bfloat16, dev, seed=11)
    g = torch.Generator("cpu").manual_seed(3)
    Lp = L + 37  # masks may be longer than the KV sequence
    if shape == "1d":
        mask = torch.rand(Lp, generator=g) < 0.6
    elif shape == "2d":
        mask = torch.rand(B, Lp, generator=g) < 0.6
    elif shape == "4d":
        mask = torch.rand(B, 1, 1, Lp, generator=g) < 0.6
    else:
        mask = torch.rand(1, 1, 1, Lp, generator=g) < 0.6
    mask = mask.to(dev)
    out, lse = _fd()(q, k, v, mask=mask, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v, mask=mask)
    assert max_abs(out, ref) < 2e-2
    assert max_abs(lse, ref_lse) < LSE_TOL


def test_all_ones_mask_equals_none(dev):
    q, k, v = _inputs(2, 24, 8, 999, 128, torch.bfloat16, dev, seed=2)
    mask = torch.ones(2, 999, dtype=torch.bool, device=dev)
    a = _fd()(q, k, v, mask=mask, num_splits=4)
    b = _fd()(q, k, v, num_splits=4)
    assert torch.equal(a, b)


def test_fully_masked_row_is_zero_and_legacy_nan(dev):
    from src.decode_attn import decode_attention
    B, L = 3, 500
    q, k, v = _inputs(B, 24, 8, L, 128, torch.bfloat16, dev, seed=4)
    mask = torch.ones(B, 1, 1, L, dtype=torch.bool)
    mask[1] = False
    mask = mask.to(dev)
    out, lse = _fd()(q, k, v, mask=mask, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v, mask=mask)
    assert torch.all(out[1] == 0)
    assert torch.all(torch.isneginf(lse[1]))
    assert max_abs(out, ref) < 2e-2
    legacy = decode_attention(q, k, v, mask=mask)
    assert torch.all(torch.isnan(legacy[1]))
    assert max_abs(legacy[0], ref[0]) < 2e-2 and max_abs(legacy[2], ref[2]) < 2e-2


def test_seq_lens_never_reads_beyond_length(dev):
    """Slots >= seq_lens[b] hold NaN; a single read of one would poison out."""
    B, Hq, Hkv, T, D = 5, 24, 8, 2048, 128
    q, k, v = _inputs(B, Hq, Hkv, T, D, torch.bfloat16, dev, seed=7)
    lens = torch.tensor([1, 17, 1024, 1500, 2048], dtype=torch.int64)
    k = k.clone()
    v = v.clone()
    for b in range(B):
        k[b, :, lens[b]:] = float("nan")
        v[b, :, lens[b]:] = float("nan")
    for splits in (1, 5, 32):
        out, lse = _fd()(q, k, v, seq_lens=lens.to(dev), num_splits=splits, return_lse=True)
        assert not torch.isnan(out).any()
        ref, ref_lse = ora.decode(q, k, v, seq_lens=lens)
        assert max_abs(out, ref) < 2e-2
        assert max_abs(lse, ref_lse) < LSE_TOL


def test_length_one_returns_v0(dev):
    q, k, v = _inputs(2, 24, 8, 1, 128, torch.bfloat16, dev, seed=8)
    out = _fd()(q, k, v)
    G = 3
    expect = v[:, :, 0].repeat_interleave(G, dim=1)
    assert torch.equal(out[:, :, 0], expect)


def test_strided_q_and_cache_views(dev):
    """q as a transposed [B,S,H,D] view; k/v as layer views of a bigger cache."""
    B, Hq, Hkv, T, L, D = 2, 24, 8, 4096, 1500, 128
    xq = randn((B, 1, Hq, D), 1, torch.bfloat16, dev)
    q = xq.transpose(1, 2)
    cache = randn((3, B, Hkv, T, D), 2, torch.bfloat16, dev)
    cache_v = randn((3, B, Hkv, T, D), 3, torch.bfloat16, dev)
    k, v = cache[1, :, :, :L], cache_v[1, :, :, :L]
    out = _fd()(q, k, v)
    ref, _ = ora.decode(q, k, v)
    assert out.stride() == q.stride()
    assert max_abs(out, ref) < 2e-2


def test_config3_full_size(dev):
    """B16, 24/8, D128, T=8192, L_b ~ randint(1024, 8193)."""
    g = torch.Generator("cpu").manual_seed(0)
    lens = torch.randint(1024, 8193, (16,), generator=g)
    assert int(lens.sum()) == 96634
    q = (torch.randn((16, 24, 1, 128), generator=g)).to(torch.bfloat16)
    kc = (torch.randn((16, 8, 8192, 128), generator=g)).to(torch.bfloat16)
    vc = (torch.randn((16, 8, 8192, 128), generator=g)).to(torch.bfloat16)
    mask = torch.arange(8192)[None, :] < lens[:, None]
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    ref, ref_lse = ora.decode(q, kc, vc, seq_lens=lens)
    out_m, lse_m = _fd()(qd, kd, vd, mask=mask.to(dev), return_lse=True)
    out_s, lse_s = _fd()(qd, kd, vd, seq_lens=lens.to(dev), return_lse=True)
    for o, l in ((out_m, lse_m), (out_s, lse_s)):
        assert max_abs(o, ref) < 2e-2
        assert max_abs(l, ref_lse) < LSE_TOL


@pytest.mark.parametrize("num_splits", [16, 32, 64, 128])
def test_config4_long_context(dev, num_splits):
    """B1, L=131072, 24/8, D128 (beyond the reference's cap)."""
    q, k, v = _inputs(1, 24, 8, 131072, 128, torch.bfloat16, dev, seed=0)
    out, lse = _fd()(q, k, v, num_splits=num_splits, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v)
    assert max_abs(out, ref) < 2e-2
    assert max_abs(lse, ref_lse) < LSE_TOL


@pytest.mark.parametrize("D,base,rems", [
    (64, 1024, (0, 1, 127, 128, 129, 256, 257, 300, 511)),   # one block: 16 waves x 8 rows
    (128, 512, (0, 1, 63, 64, 65, 128, 129, 200, 255)),      # 16 waves x 4 rows
])
def test_split_pass_remainders(dev, D, base, rems):
    """Key ranges that end exactly on a 4-row-group pass, one or two groups
    past it (finished in one-group passes) and more (one more clamped pass):
    every branch of the split loop against the oracle, with NaN in every slot
    at or past the length so that any read beyond it would show."""
    B, Hq, Hkv = len(rems), 4, 1
    T = base + 512
    q, k, v = _inputs(B, Hq, Hkv, T, D, torch.bfloat16, dev, seed=11)
    lens = torch.tensor([base + r for r in rems], dtype=torch.int64)
    k, v = k.clone(), v.clone()
    for b in range(B):
        k[b, :, lens[b]:] = float("nan")
        v[b, :, lens[b]:] = float("nan")
    for splits in (1, 3):
        out, lse = _fd()(q, k, v, seq_lens=lens.to(dev), num_splits=splits, return_lse=True)
        ref, ref_lse = ora.decode(q, k, v, seq_lens=lens)
        assert not torch.isnan(out).any(), (D, splits)
        assert max_abs(out, ref) < 2e-2, (D, splits)
        assert max_abs(lse, ref_lse) < LSE_TOL, (D, splits)


@pytest.mark.parametrize("D,L,splits", [(128, 9000, 1), (128, 9000, 4), (64, 5000, 2), (64, 300, 3)])
def test_mask_excluded_rows_are_not_read(dev, D, L, splits):
    """The mask path streams only the rows the mask keeps: K/V rows it excludes
    hold NaN and must not reach the output (the reference loads them and would
    propagate the NaN through 0 * V).  L = 9000 with one split crosses the
    4096-row mask windows; a window with every row excluded is included."""
    B, Hq, Hkv = 3, 8, 2
    q, k, v = _inputs(B, Hq, Hkv, L, D, torch.bfloat16, dev, seed=21)
    g = torch.Generator().manual_seed(22)
    mask = torch.rand((B, L), generator=g) < 0.5
    mask[1, : min(L, 4500)] = False            # whole window(s) excluded
    mask[2] = False
    mask[2, L - 1] = True                      # a single key, the last one
    kc, vc = k.clone(), v.clone()
    keep = mask.to(dev)[:, None, :, None]
    k = torch.where(keep, k, torch.full_like(k, float("nan")))
    v = torch.where(keep, v, torch.full_like(v, float("nan")))
    out, lse = _fd()(q, k, v, mask=mask.to(dev), num_splits=splits, return_lse=True)
    assert not torch.isnan(out).any()
    ref, ref_lse = ora.decode(q, kc, vc, mask=mask)
    assert max_abs(out, ref) < 2e-2
    empty = torch.isneginf(ref_lse)            # rows the mask empties entirely: -inf
    assert torch.equal(torch.isneginf(lse.cpu()), empty)
    assert max_abs(lse.cpu()[~empty], ref_lse[~empty]) < LSE_TOL


def test_row_stride_past_buffer_span(dev):
    """K/V rows 600 KB apart (a view into a larger cache): past the span the
    buffer-offset loads cover, the element-load path serves the call."""
    B, Hq, Hkv, L, D, stride = 1, 4, 1, 40, 64, 300_000
    g = torch.Generator().manual_seed(41)
    q = torch.randn((B, Hq, 1, D), generator=g).to(torch.bfloat16).to(dev)
    kbuf = torch.randn((L * stride,), generator=g).to(torch.bfloat16).to(dev)
    vbuf = torch.randn((L * stride,), generator=g).to(torch.bfloat16).to(dev)
    k = kbuf.as_strided((B, Hkv, L, D), (L * stride, L * stride, stride, 1))
    v = vbuf.as_strided((B, Hkv, L, D), (L * stride, L * stride, stride, 1))
    for splits in (1, 4):
        out, lse = _fd()(q, k, v, num_splits=splits, return_lse=True)
        ref, ref_lse = ora.decode(q, k.contiguous(), v.contiguous())
        assert max_abs(out, ref) < 2e-2
        assert max_abs(lse, ref_lse) < LSE_TOL


@pytest.mark.parametrize("splits", [1, 3])
def test_mask_window_bounds(dev, splits):
    """Each 4096-row mask window streams only rows between its first and last
    selected key: runs that end on a window boundary, start and end inside
    windows, a single selected key at a window start, and a run through the
    last row, with NaN in every row the mask excludes."""
    B, Hq, Hkv, L, D = 4, 8, 2, 9000, 128
    q, k, v = _inputs(B, Hq, Hkv, L, D, torch.bfloat16, dev, seed=31)
    mask = torch.zeros((B, L), dtype=torch.bool)
    for b, (lo, hi) in enumerate([(0, 4096), (100, 4200), (4096, 4097), (8191, 9000)]):
        mask[b, lo:hi] = True
    kc, vc = k.clone(), v.clone()
    keep = mask.to(dev)[:, None, :, None]
    k = torch.where(keep, k, torch.full_like(k, float("nan")))
    v = torch.where(keep, v, torch.full_like(v, float("nan")))
    out, lse = _fd()(q, k, v, mask=mask.to(dev), num_splits=splits, return_lse=True)
    assert not torch.isnan(out).any()
    ref, ref_lse = ora.decode(q, kc, vc, mask=mask)
    assert max_abs(out, ref) < 2e-2
    assert max_abs(lse, ref_lse) < LSE_TOL


@pytest.mark.parametrize("B", [2, 3, 64, 65])
def test_seq_lens_rows_dealt_by_length(dev, B):
    """With seq_lens and 2 <= B <= 64 the split kernel deals its grid rows by
    sequence length (longest first, then shortest first); B = 65 keeps the
    plain order.  Ties, empty sequences and lengths past the capacity
    (clamped to it) must all land on their own rows: every row is checked
    against the oracle, and a bit-identical rerun with the lengths permuted
    with the batch shows the mapping is a permutation."""
    T, Hq, Hkv, D = 320, 8, 2, 64
    g = torch.Generator("cpu").manual_seed(B)
    lens = torch.randint(0, T + 1, (B,), generator=g)
    lens[0] = lens[-1]                       # a tie
    lens[1] = 0                              # an empty sequence
    if B > 2:
        lens[2] = T + 50                     # past the capacity: clamped to T
    q, k, v = _inputs(B, Hq, Hkv, T, D, torch.bfloat16, dev, seed=7)
    out, lse = _fd()(q, k, v, seq_lens=lens.to(dev), num_splits=2, return_lse=True)
    ref, ref_lse = ora.decode(q.cpu(), k.cpu(), v.cpu(), seq_lens=lens.clamp(max=T))
    nonempty = lens > 0
    assert max_abs(out[nonempty], ref[nonempty]) < TOL[torch.bfloat16]
    assert max_abs(lse[nonempty], ref_lse[nonempty]) < LSE_TOL
    assert torch.all(out[~nonempty] == 0)
    assert torch.all(torch.isneginf(lse[~nonempty]))
    perm = torch.randperm(B, generator=g)
    pd = perm.to(dev)
    out_p, lse_p = _fd()(q[pd].contiguous(), k[pd].contiguous(), v[pd].contiguous(),
                         seq_lens=lens[perm].to(dev), num_splits=2, return_lse=True)
    assert torch.equal(out_p, out[pd])
    assert torch.equal(lse_p, lse[pd])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [8, 48, 80, 96, 112, 160, 192, 200])
def test_decode_head_dims_not_powers_of_two(dev, D, dtype):
    """Any head_dim <= 256 (the reference pads to the next power of two and
    masks d < HEAD_DIM, src/flash_decode.py:55-61, :274-277): head dims that
    fill whole 16-byte chunks run the chunk loads with the lanes past them
    idle; through the default split count, one split, 40 splits, per-sequence
    lengths and a mask."""
    q, k, v = _inputs(2, 6, 2, 515, D, dtype, dev, seed=19)
    sl = torch.tensor([515, 77], dtype=torch.int64, device=dev)
    mask = (torch.rand(2, 515, generator=torch.Generator().manual_seed(5)) < 0.5).to(dev)
    for kw, ref_kw in (({}, {}), ({"num_splits": 1}, {}), ({"num_splits": 40}, {}),
                       ({"seq_lens": sl}, {"seq_lens": sl}), ({"mask": mask}, {"mask": mask}),
                       ({"mask": mask, "num_splits": 3}, {"mask": mask})):
        out, lse = _fd()(q, k, v, return_lse=True, **kw)
        ref, ref_lse = ora.decode(q, k, v, **ref_kw)
        assert out.shape == q.shape
        assert max_abs(out, ref) < TOL[dtype], (D, dtype, kw.keys())
        assert max_abs(lse, ref_lse) < LSE_TOL, (D, dtype, kw.keys())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [1, 3, 4, 36, 100, 130, 255, 256])
def test_decode_element_loads(dev, D, dtype):
    """Head dims whose rows are not whole 16-byte chunks (and rows that are
    not 16-byte aligned: a [..., 1:] view of wider rows) are read element by
    element; D = 256 through such a view checks the same path at full width."""
    B, Hq, Hkv, L = 3, 8, 2, 700
    g = torch.Generator().manual_seed(D)
    q = torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(dev)
    kw_ = torch.randn((B, Hkv, L, D + 1), generator=g).to(dtype).to(dev)
    vw_ = torch.randn((B, Hkv, L, D + 1), generator=g).to(dtype).to(dev)
    k, v = kw_[..., 1:], vw_[..., 1:]
    sl = torch.tensor([700, 1, 333], dtype=torch.int64, device=dev)
    for kw, ref_kw in (({}, {}), ({"num_splits": 1}, {}), ({"num_splits": 7}, {}),
                       ({"seq_lens": sl}, {"seq_lens": sl})):
        out, lse = _fd()(q, k, v, return_lse=True, **kw)
        ref, ref_lse = ora.decode(q, k, v, **ref_kw)
        assert max_abs(out, ref) < TOL[dtype], (D, dtype, kw.keys())
        assert max_abs(lse, ref_lse) < LSE_TOL, (D, dtype, kw.keys())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("path", ["seq_lens", "mask"])
@pytest.mark.parametrize("B", [8, 16])
def test_pipelined_last_pass_lengths(dev, dtype, path, B):
    """Config 5's per-layer shape (B8 32/8 D64, 4 splits: one block per CU, the
    software-pipelined loop at 8 waves, 256 rows per pass); B16 doubles the
    grid (two blocks per CU: the pipelined loop at 4 waves for seq_lens, the
    single-buffered one for the mask).  The sequence lengths leave each split
    a last pass of one row (L = 1), 16 rows (4097: one row slot at 8 waves),
    80 (4353: two slots), 144 (4609: a full pass), none (4096: whole passes),
    240 (4000) and short splits (63, 130); every case against the oracle."""
    Hq, Hkv, D, T, S = 32, 8, 64, 4736, 4
    q, k, v = _inputs(B, Hq, Hkv, T, D, dtype, dev, seed=41)
    lens = torch.tensor([4097, 4353, 4609, 4096, 4000, 1, 63, 130] * (B // 8))
    if path == "seq_lens":
        out, lse = _fd()(q, k, v, num_splits=S, seq_lens=lens.to(dev), return_lse=True)
    else:
        mask = (torch.arange(T)[None, :] < lens[:, None]).to(dev)
        out, lse = _fd()(q, k, v, num_splits=S, mask=mask, return_lse=True)
    ref, ref_lse = ora.decode(q, k, v, seq_lens=lens)
    assert max_abs(out, ref) < TOL[dtype], path
    assert max_abs(lse, ref_lse) < LSE_TOL, path


@pytest.mark.parametrize("B,Hq,Hkv,L,D,S", [
    (8, 32, 8, 4097, 64, 4),        # config 5's per-layer shape: in-launch combine
    (2, 8, 2, 999, 128, 8),         # few groups, 8 splits: in-launch combine
    (4, 8, 8, 5000, 128, 2),        # MHA, 2 splits widened to 4: in-launch combine
    (16, 24, 8, 3000, 128, 4),      # config 3's heads, 512 blocks: two launches
    (1, 24, 8, 20000, 128, 32),     # config 4-like, 32 splits: two launches
    (3, 8, 2, 999, 96, 16),         # padded head_dim: two launches
    (2, 6, 2, 2000, 64, 200),       # many splits: two launches (block combine)
])
def test_in_launch_combine_matches_combine_kernel(dev, monkeypatch, B, Hq, Hkv, L, D, S):
    """With the library's arrival counters, calls whose split blocks are few
    and short run the LSE combine inside the split launch (the last split of
    each group combines); it gives bit for bit what the separate combine
    kernel gives whenever that kernel is the wave-per-row one (<= 16 splits,
    >= 64 rows), and the oracle's result otherwise; three calls in a row check
    that every call leaves its arrival counters at zero.  Other shapes take
    the two launches either way."""
    from src import _lib
    q, k, v = _inputs(B, Hq, Hkv, L, D, torch.bfloat16, dev, seed=31)
    g = torch.Generator().manual_seed(S)
    sl = torch.randint(1, L + 1, (B,), generator=g).to(dev)
    ref, ref_lse = ora.decode(q, k, v, seq_lens=sl)
    fused = [_fd()(q, k, v, num_splits=S, seq_lens=sl, return_lse=True) for _ in range(3)]
    with monkeypatch.context() as m:
        m.setattr(_lib, "arrive_counters", lambda *a: None)
        two = _fd()(q, k, v, num_splits=S, seq_lens=sl, return_lse=True)
    eff = int(_lib.load().mi_decode_effective_splits(B, Hq, Hkv, L, D, S))
    for out, lse in fused:
        assert torch.equal(out, fused[0][0]) and torch.equal(lse, fused[0][1])
        assert max_abs(out, ref) < 2e-2
        assert max_abs(lse, ref_lse) < LSE_TOL
    if eff <= 16 and B * Hq >= 64:
        assert torch.equal(fused[0][0], two[0]) and torch.equal(fused[0][1], two[1])
    else:
        assert max_abs(two[0], ref) < 2e-2 and max_abs(two[1], ref_lse) < LSE_TOL


def test_in_launch_combine_on_two_streams(dev):
    """Calls on two streams at once use separate arrival counters (one slab
    per stream): interleaved, unsynchronised calls on both stay correct."""
    q, k, v = _inputs(8, 24, 8, 4096, 128, torch.bfloat16, dev, seed=41)
    q2, k2, v2 = _inputs(8, 24, 8, 4096, 128, torch.bfloat16, dev, seed=42)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for i in range(6):
        st, (qq, kk, vv) = (s1, (q, k, v)) if i % 2 == 0 else (s2, (q2, k2, v2))
        with torch.cuda.stream(st):
            outs.append(_fd()(qq, kk, vv, num_splits=8))
    torch.cuda.synchronize()
    ref1, _ = ora.decode(q, k, v)
    ref2, _ = ora.decode(q2, k2, v2)
    for i, o in enumerate(outs):
        assert max_abs(o, ref1 if i % 2 == 0 else ref2) < 2e-2, i


def test_in_launch_combine_under_graph_replay(dev):
    """A captured flash_decode (seq_lens, several splits) replayed at changing
    lengths, with eager calls on the same stream between the replays, matches
    the eager call every time."""
    B, Hq, Hkv, T, D = 4, 24, 8, 4096, 128
    q, k, v = _inputs(B, Hq, Hkv, T, D, torch.bfloat16, dev, seed=43)
    sl = torch.full((B,), T, dtype=torch.int64, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _fd()(q, k, v, seq_lens=sl, num_splits=6)          # warm-up on the capture side
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = _fd()(q, k, v, seq_lens=sl, num_splits=6)
    for lens in ([4096, 1, 2000, 17], [33, 4095, 4096, 1024], [1, 1, 1, 1]):
        sl.copy_(torch.tensor(lens, dtype=torch.int64))
        graph.replay()
        eager = _fd()(q, k, v, seq_lens=sl, num_splits=6)
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), lens
        ref, _ = ora.decode(q, k, v, seq_lens=sl)
        assert max_abs(out_g, ref) < 2e-2, lens
