"""CPU: the Python entry points raise the reference's exceptions and messages
for bad arguments (src/flash_decode.py:215-285, src/kv_cache.py:39-46,
src/cuda_graph.py:10-11) before anything reaches the GPU."""
import pytest
import torch


def _fd():
    from src.flash_decode import flash_decode
    return flash_decode


def _t(*shape, dtype=torch.bfloat16):
    return torch.zeros(shape, dtype=dtype)


@pytest.mark.parametrize("q,k,v,exc,msg", [
    (_t(2, 8, 128), _t(2, 8, 5, 128), _t(2, 8, 5, 128), ValueError, "rank-4"),
    (_t(2, 8, 2, 128), _t(2, 8, 5, 128), _t(2, 8, 5, 128), ValueError, "query_len=1, got 2"),
    (_t(2, 8, 1, 128), _t(2, 8, 5, 128), _t(2, 8, 6, 128), ValueError, "k and v shapes must match"),
    (_t(2, 8, 1, 128), _t(3, 8, 5, 128), _t(3, 8, 5, 128), ValueError, "batch size and head dimension"),
    (_t(2, 8, 1, 64), _t(2, 8, 5, 128), _t(2, 8, 5, 128), ValueError, "batch size and head dimension"),
    (_t(2, 8, 1, 128), _t(2, 8, 0, 128), _t(2, 8, 0, 128), ValueError, "must not be empty"),
    (_t(2, 12, 1, 128), _t(2, 8, 5, 128), _t(2, 8, 5, 128), ValueError, "divisible by KV heads"),
    (_t(2, 8, 1, 128), _t(2, 8, 5, 128), _t(2, 8, 5, 128), ValueError, "requires CUDA tensors"),
])
def test_flash_decode_argument_errors(q, k, v, exc, msg):
    with pytest.raises(exc, match=msg):
        _fd()(q, k, v)


def test_mask_strides_rules():
    from src.flash_decode import _mask_strides
    with pytest.raises(TypeError, match="torch.bool"):
        _mask_strides(torch.zeros(10), 2, 10)
    with pytest.raises(ValueError, match="at least one dimension"):
        _mask_strides(torch.tensor(True), 2, 10)
    with pytest.raises(ValueError, match="shorter"):
        _mask_strides(torch.ones(9, dtype=torch.bool), 2, 10)
    with pytest.raises(ValueError, match="batch dimension must be 1 or 2"):
        _mask_strides(torch.ones(3, 10, dtype=torch.bool), 2, 10)
    with pytest.raises(ValueError, match="except batch and KV length must be 1"):
        _mask_strides(torch.ones(2, 2, 1, 10, dtype=torch.bool), 2, 10)
    assert _mask_strides(torch.ones(12, dtype=torch.bool), 2, 10) == (0, 1)
    assert _mask_strides(torch.ones(2, 12, dtype=torch.bool), 2, 10) == (12, 1)
    assert _mask_strides(torch.ones(1, 1, 1, 12, dtype=torch.bool), 2, 10) == (0, 1)
    assert _mask_strides(torch.ones(2, 1, 1, 12, dtype=torch.bool), 2, 10) == (12, 1)


def test_kv_cache_position_errors():
    from src.config import ModelArgs
    from src.kv_cache import KVCache
    kv = KVCache(ModelArgs(dim=64, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=8,
                           device="cpu"), dtype=torch.bfloat16)
    assert kv.k.shape == (1, 1, 1, 8, 32)
    with pytest.raises(ValueError, match="1D tensor"):
        kv.update_positions(0, torch.zeros(1, 1, dtype=torch.long), _t(1, 1, 1, 32), _t(1, 1, 1, 32))
    with pytest.raises(ValueError, match="length mismatch"):
        kv.update_positions(0, torch.zeros(2, dtype=torch.long), _t(1, 1, 1, 32), _t(1, 1, 1, 32))


def test_model_args_defaults_are_llama_3_2_1b():
    from src.config import ModelArgs
    a = ModelArgs()
    assert (a.dim, a.n_layers, a.n_heads, a.n_kv_heads, a.vocab_size, a.hidden_dim) == \
        (2048, 16, 32, 8, 128256, 8192)
    assert (a.norm_eps, a.max_batch_size, a.max_seq_len, a.rope_theta) == (1e-5, 1, 4096, 500000.0)


def test_small_m_w8a16_routing_rule():
    """Which small-M products W8A16Linear sends to the decode-step projection
    kernel (the rest run the GEMV kernel): bf16/fp16 x with unit k stride and
    16-byte rows, scales in x's dtype, K in the kernel's set, <= 16 rows."""
    import torch
    from src.quant_linear import _fused_gemv_ok
    x = torch.zeros(8, 2048, dtype=torch.bfloat16)
    w = torch.zeros(2048, 2048, dtype=torch.int8)
    s = torch.zeros(2048, dtype=torch.bfloat16)
    assert _fused_gemv_ok(x, w, s)
    assert _fused_gemv_ok(x.half(), w, s.half())
    assert not _fused_gemv_ok(x, w, s.float())                           # fp32 scales
    assert not _fused_gemv_ok(x[:, :2000], w[:, :2000], s)                # K not served
    assert not _fused_gemv_ok(torch.zeros(17, 2048, dtype=torch.bfloat16), w, s)
    assert not _fused_gemv_ok(x.float(), w, s.float())                    # fp32 x
    assert not _fused_gemv_ok(torch.zeros(2048, 8, dtype=torch.bfloat16).t(), w, s)  # k stride


@pytest.mark.parametrize("shape,layer,msg", [
    ((3, 2, 1, 16), 0, "does not fit the cache"),     # batch above max_batch_size
    ((2, 3, 1, 16), 0, "does not fit the cache"),     # more kv heads than the cache
    ((2, 1, 1, 16), 0, "does not fit the cache"),     # fewer kv heads (slot stride differs)
    ((2, 2, 1, 32), 0, "does not fit the cache"),     # wider head_dim
    ((2, 2, 1, 8), 0, "does not fit the cache"),      # narrower head_dim
    ((2, 2, 1, 16), 2, "layer_idx 2 out of range"),   # past the last layer
])
def test_rope_and_cache_update_rejects_shapes_the_cache_does_not_hold(shape, layer, msg):
    """Checked before anything launches (the kernel would otherwise write into
    the next layer's slabs or past the allocation, src/rope.py:255-313)."""
    from src.config import ModelArgs
    from src.kv_cache import KVCache
    from src.rope import rope_and_cache_update
    args = ModelArgs(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=32, max_batch_size=2,
                     max_seq_len=8, device="cpu")
    kv = KVCache(args, dtype=torch.bfloat16)
    cos = torch.ones(1, shape[3] // 2, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=msg):
        rope_and_cache_update(_t(*shape), _t(*shape), cos, cos, kv, layer, start_pos=0)


def test_quantized_blocks_run_the_fused_prefill_classes():
    """Llama3Quantized's blocks hold QuantizedAttention / QuantizedFeedForward
    (one-launch q|k|v, SwiGLU and residual epilogues at prefill sizes), with
    the parameter names of the plain modules (the checkpoint format), and the
    plain Llama3 keeps the plain ones."""
    import torch
    from src.config import ModelArgs
    from src.model import Attention, FeedForward, Llama3
    from src.model_quantized import Llama3Quantized, QuantizedAttention, QuantizedFeedForward
    args = ModelArgs(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=64, hidden_dim=512)
    with torch.device("meta"):
        mq, mp = Llama3Quantized(args), Llama3(args)
    for layer in mq.layers:
        assert isinstance(layer.attention, QuantizedAttention)
        assert isinstance(layer.feed_forward, QuantizedFeedForward)
    for layer in mp.layers:
        assert type(layer.attention) is Attention and type(layer.feed_forward) is FeedForward
    kq, kp = set(mq.state_dict()), set(mp.state_dict())
    assert kp <= kq and all(k.endswith(".scales") for k in kq - kp)
