"""GPU parity of checkpoint loading (src/loader.py), end to end.

A Hugging Face Llama checkpoint (random init from transformers' own
LlamaForCausalLM, norms perturbed, bf16) is loaded by build_model_from_weights
and run through the engine's prefill and one decode step over its KV cache (as
main.py runs it: the engine, like the reference, rotates K inside the cache
update, src/model.py:57-76); the reference forward is transformers'
LlamaForCausalLM in fp32 on the CPU with the same bf16-rounded weights.  This
pins the name remap, the gate/up/down roles, GQA head grouping, the RoPE
convention and llama3 frequency scaling, tied embeddings and the final norm
against an implementation the engine shares no code with.  Bars: with fp32
activations (the engine's fp32 kernels) logits within 1e-3 of the logit scale
-- any semantic mismatch is far above that; with bf16 activations within 8e-2
(every projection, norm, residual and attention output rounded to bf16 through
2 layers); W8A16 weights and scales bit-exact with the CPU oracle's quantiser,
and the W8A16 engine (bf16 activations) within 8e-2 of transformers running the
dequantised weights (q * s) in fp32.
"""
import numpy as np
import pytest
import torch

from oracle import quant as oq

pytestmark = pytest.mark.gpu

SHAPE = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, hidden_dim=512)
LLAMA3_ROPE = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
               "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def _hf_model(tied, rope_scaling, seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    rp = {"rope_type": "default", "rope_theta": 500000.0}
    if rope_scaling:
        rp = dict(rope_scaling, rope_theta=500000.0)
    cfg = LlamaConfig(hidden_size=SHAPE["dim"], intermediate_size=SHAPE["hidden_dim"],
                      num_hidden_layers=SHAPE["n_layers"], num_attention_heads=SHAPE["n_heads"],
                      num_key_value_heads=SHAPE["n_kv_heads"], vocab_size=SHAPE["vocab_size"],
                      max_position_embeddings=131072, rms_norm_eps=1e-5, tie_word_embeddings=tied,
                      rope_parameters=rp)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            p.copy_(p.to(torch.bfloat16).float())        # the checkpoint's values exactly
    return m


def _checkpoint(tmp_path, m, tied):
    from safetensors.torch import save_file
    sd = {k: v.detach().to(torch.bfloat16).contiguous() for k, v in m.state_dict().items()
          if "rotary" not in k}
    if tied:
        sd.pop("lm_head.weight", None)
    p = tmp_path / "model.safetensors"
    save_file(sd, str(p))
    return p, sd


def _args(dev, rope_scaling):
    from src.config import ModelArgs
    return ModelArgs(max_batch_size=2, max_seq_len=64, device=str(dev), rope_scaling=rope_scaling,
                     **SHAPE)


def _prefill_and_decode(model, args, tokens, dev, dtype):
    """Engine logits of every prompt position, then of one decoded token."""
    from src.kv_cache import KVCache
    kv = KVCache(args, dtype=dtype)
    S = tokens.shape[1] - 1
    with torch.no_grad():
        pre = model(tokens[:, :S].to(dev), start_pos=0, kv_cache=kv, return_all_logits=True)
        dec = model(tokens[:, S:].to(dev), start_pos=S, kv_cache=kv)
    return pre, dec


def _close(a, b, tol):
    a, b = a.float().cpu(), b.float().cpu()
    scale = float(b.abs().max()) + 1e-6
    err = float((a - b).abs().max())
    assert err < tol * scale, (err, scale)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 8e-2)])
@pytest.mark.parametrize("tied,rope_scaling", [(False, None), (True, LLAMA3_ROPE)])
def test_hf_checkpoint_prefill_matches_transformers(tmp_path, dev, tied, rope_scaling, dtype, tol):
    from src.loader import build_model_from_weights
    from src.model import Llama3
    hf = _hf_model(tied, rope_scaling)
    path, _ = _checkpoint(tmp_path, hf, tied)
    model, rep = build_model_from_weights(Llama3, _args(dev, rope_scaling), path, str(dev),
                                          dtype=dtype)
    assert rep["missing"] == []
    args = _args(dev, rope_scaling)
    tokens = torch.randint(0, SHAPE["vocab_size"], (2, 41), generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        ref = hf(tokens).logits
    pre, dec = _prefill_and_decode(model, args, tokens, dev, dtype)
    assert pre.shape == ref[:, :40].shape and pre.dtype == dtype
    _close(pre, ref[:, :40], tol)
    _close(dec.reshape(2, -1), ref[:, 40], tol)
    if tied:
        assert model.output.weight.data_ptr() == model.tok_embeddings.weight.data_ptr()


def test_w8a16_load_is_bit_exact_and_matches_dequantised_reference(tmp_path, dev):
    from src.loader import build_model_from_weights
    from src.model import Llama3
    from src.quant_utils import get_transformer_linear_names
    from src.loader import _to_hf_name
    hf = _hf_model(True, LLAMA3_ROPE, seed=3)
    path, sd = _checkpoint(tmp_path, hf, True)
    model, rep = build_model_from_weights(Llama3, _args(dev, LLAMA3_ROPE), path, str(dev),
                                          dtype=torch.bfloat16, quantization="w8a16")
    assert type(model).__name__ == "Llama3Quantized" and rep["missing"] == []
    hf_params = dict(hf.named_parameters())
    with torch.no_grad():
        for i in range(SHAPE["n_layers"]):
            for mod in get_transformer_linear_names():
                key = f"layers.{i}.{mod}.weight"
                lin = model.get_submodule(f"layers.{i}.{mod}")
                rq, rs = oq.quantize_per_channel(sd[_to_hf_name(key)].float().numpy(), "bfloat16")
                assert lin.weight.dtype == torch.int8 and lin.scales.dtype == torch.bfloat16
                assert np.array_equal(lin.weight.cpu().numpy(), rq), key
                assert np.array_equal(lin.scales.float().cpu().numpy(), rs), key
                # the reference model runs the dequantised weight in fp32
                hf_params[_to_hf_name(key)].copy_(torch.from_numpy(rq).float() * torch.from_numpy(rs))
    tokens = torch.randint(0, SHAPE["vocab_size"], (2, 34), generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        ref = hf(tokens).logits
    pre, dec = _prefill_and_decode(model, _args(dev, LLAMA3_ROPE), tokens, dev, torch.bfloat16)
    _close(pre, ref[:, :33], 8e-2)
    _close(dec.reshape(2, -1), ref[:, 33], 8e-2)
