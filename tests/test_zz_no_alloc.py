"""GPU: mi_flash_decode_noalloc (split partials in the library's own device
array, nothing allocated per call) gives the same out and LSE as
mi_flash_decode with a caller workspace, bit for bit (same kernels, same split
count), on two calls in a row, the second smaller than the first; a request
whose partials do not fit the array is refused before anything launches."""
import math

import pytest
import torch

from helpers import randn

pytestmark = pytest.mark.gpu


def _noalloc(q, k, v, *, mask=None, seq_lens=None, num_splits):
    from src import _lib
    from src.flash_decode import _mask_strides
    B, Hq, _, D = q.shape
    _, Hkv, L, _ = k.shape
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq), device=q.device, dtype=torch.float32)
    msb, msl = (0, 0) if mask is None else _mask_strides(mask, B, L)
    st = _lib.load().mi_flash_decode_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(mask), msb, msl, _lib.ptr(seq_lens),
        out.data_ptr(), lse.data_ptr(), B, Hq, Hkv, L, D, num_splits,
        q.stride(0), q.stride(1), q.stride(3), k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1), out.stride(3),
        1.0 / math.sqrt(D), 0, _lib.dtype_code(q.dtype), _lib.stream_of(q))
    return st, out, lse


def _case(dev, B, Hq, Hkv, L, D, splits, seed, use_mask):
    from src.flash_decode import flash_decode
    q = randn((B, Hq, 1, D), seed, device=dev)
    k = randn((B, Hkv, L, D), seed + 1, device=dev)
    v = randn((B, Hkv, L, D), seed + 2, device=dev)
    g = torch.Generator().manual_seed(seed + 3)
    lens = torch.randint(1, L + 1, (B,), generator=g)
    kw = {}
    if use_mask:
        kw["mask"] = (torch.arange(L)[None, :] < lens[:, None]).to(dev)
    else:
        kw["seq_lens"] = lens.to(dev)
    ref, ref_lse = flash_decode(q, k, v, num_splits=splits, return_lse=True, **kw)
    st, out, lse = _noalloc(q, k, v, num_splits=splits, **kw)
    torch.cuda.synchronize()
    assert st == 0
    assert torch.equal(out, ref)
    assert torch.equal(lse, ref_lse)


def test_noalloc_matches_workspace_entry_point_twice(dev):
    """Larger call first (config 3 head layout, seq_lens), then a smaller one
    (mask path, D 64): the second must not see the first call's partials."""
    print("noalloc case 1: B16 Hq24 Hkv8 L4096 D128 splits 8 seq_lens", flush=True)
    _case(dev, 16, 24, 8, 4096, 128, 8, 0, use_mask=False)
    print("noalloc case 2: B2 Hq8 Hkv2 L300 D64 splits 3 mask", flush=True)
    _case(dev, 2, 8, 2, 300, 64, 3, 10, use_mask=True)
    print("noalloc case 3: B1 Hq24 Hkv8 L131072 D128 splits 128 seq_lens", flush=True)
    _case(dev, 1, 24, 8, 131072, 128, 128, 20, use_mask=False)


def test_noalloc_rejects_partials_beyond_the_scratch(dev):
    """B*Hq*S*(D+2)*4 bytes above the 16 MiB array: refused, nothing launched."""
    q = torch.zeros((64, 32, 1, 128), device=dev, dtype=torch.bfloat16)
    k = torch.zeros((64, 8, 4096, 128), device=dev, dtype=torch.bfloat16)
    st, _, _ = _noalloc(q, k, k, num_splits=64)        # 64*32*64*130*4 = 68 MB
    assert st == -2
    from src import _lib
    assert "scratch" in _lib.load().mi_last_error().decode()


def test_noalloc_under_graph_capture(dev):
    """The stated use: two calls captured in one graph (the entry point
    allocates nothing; the two calls share the library's array one after the
    other),
    replayed three times at changing lengths with eager work on the stream in
    between; every replay matches flash_decode with a caller workspace bit
    for bit."""
    from src.flash_decode import flash_decode
    print("noalloc graph: B8 Hq24 Hkv8 L2048 D128 splits 4 + B2 Hq8 Hkv2 L500 D64 splits 3",
          flush=True)
    qa, ka, va = (randn((8, 24, 1, 128), 50, device=dev), randn((8, 8, 2048, 128), 51, device=dev),
                  randn((8, 8, 2048, 128), 52, device=dev))
    qb, kb, vb = (randn((2, 8, 1, 64), 53, device=dev), randn((2, 2, 500, 64), 54, device=dev),
                  randn((2, 2, 500, 64), 55, device=dev))
    sla = torch.full((8,), 2048, dtype=torch.int64, device=dev)
    slb = torch.full((2,), 500, dtype=torch.int64, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st_a, out_a, lse_a = _noalloc(qa, ka, va, seq_lens=sla, num_splits=4)
        st_b, out_b, lse_b = _noalloc(qb, kb, vb, seq_lens=slb, num_splits=3)
    assert st_a == 0 and st_b == 0
    for la, lb in (([2048, 1, 700, 2047, 5, 1024, 1500, 3], [500, 17]),
                   ([1] * 8, [1, 499]), ([999] * 8, [250, 250])):
        sla.copy_(torch.tensor(la))
        slb.copy_(torch.tensor(lb))
        graph.replay()
        ra, rla = flash_decode(qa, ka, va, seq_lens=sla, num_splits=4, return_lse=True)
        rb, rlb = flash_decode(qb, kb, vb, seq_lens=slb, num_splits=3, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(out_a, ra) and torch.equal(lse_a, rla), la
        assert torch.equal(out_b, rb) and torch.equal(lse_b, rlb), lb
