"""Checkpoint loader (src/loader.py) and quantisation helpers (src/quant_utils.py),
host side: no GPU needed.

Checkpoints are written in Hugging Face Llama names and shapes taken from
transformers' own LlamaForCausalLM (the naming authority the reference's remap
table targets), so the remap is checked against an independent source.  The
forward-pass equivalence with transformers and the W8A16 quantisation on the
device are in tests/test_gpu_loader.py.
"""
import math

import pytest
import torch

TINY = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, hidden_dim=160,
            max_seq_len=32)


def _hf_state(seed=0, tied=False):
    """Random HF-named state dict of the TINY shape (bf16)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=TINY["dim"], intermediate_size=TINY["hidden_dim"],
                      num_hidden_layers=TINY["n_layers"], num_attention_heads=TINY["n_heads"],
                      num_key_value_heads=TINY["n_kv_heads"], vocab_size=TINY["vocab_size"],
                      max_position_embeddings=131072, tie_word_embeddings=tied)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg)
    sd = {k: v.detach().to(torch.bfloat16).contiguous().clone() for k, v in m.state_dict().items()}
    sd = {k: v for k, v in sd.items() if "rotary" not in k}
    g = torch.Generator().manual_seed(seed + 1)
    for k in sd:                      # distinct values everywhere (norms are all-ones at init)
        sd[k] = torch.randn(sd[k].shape, generator=g).to(torch.bfloat16)
    if tied:
        sd.pop("lm_head.weight", None)
    return sd


def _save(tmp_path, sd, name="model.safetensors"):
    from safetensors.torch import save_file
    p = tmp_path / name
    save_file(sd, str(p))
    return p


def _args():
    from src.config import ModelArgs
    return ModelArgs(device="cpu", **TINY)


@pytest.mark.parametrize("tied", [False, True])
def test_hf_checkpoint_loads_every_parameter(tmp_path, tied):
    from src.loader import build_model_from_weights
    from src.model import Llama3
    sd = _hf_state(0, tied)
    model, rep = build_model_from_weights(Llama3, _args(), _save(tmp_path, sd), "cpu",
                                          dtype=torch.bfloat16)
    assert rep["missing"] == [] and rep["unexpected"] == []
    params = dict(model.named_parameters())
    n_model = len(model.state_dict())
    assert rep["loaded"] == n_model
    # every engine parameter is one checkpoint tensor, and distinct parameters
    # are distinct tensors (a bijection), except the tied output head
    seen = {}
    for name, p in model.state_dict().items():
        hits = [k for k, v in sd.items() if v.shape == p.shape and torch.equal(v, p)]
        assert len(hits) == 1, (name, hits)
        seen.setdefault(hits[0], []).append(name)
    if tied:
        assert sorted(seen["model.embed_tokens.weight"]) == ["output.weight", "tok_embeddings.weight"]
    else:
        assert seen["lm_head.weight"] == ["output.weight"]
    # the Hugging Face roles of the projections (gate = w1, up = w3, down = w2)
    L = "model.layers.1."
    assert torch.equal(params["layers.1.attention.wq.weight"], sd[L + "self_attn.q_proj.weight"])
    assert torch.equal(params["layers.1.attention.wk.weight"], sd[L + "self_attn.k_proj.weight"])
    assert torch.equal(params["layers.1.attention.wv.weight"], sd[L + "self_attn.v_proj.weight"])
    assert torch.equal(params["layers.1.attention.wo.weight"], sd[L + "self_attn.o_proj.weight"])
    assert torch.equal(params["layers.1.feed_forward.w1.weight"], sd[L + "mlp.gate_proj.weight"])
    assert torch.equal(params["layers.1.feed_forward.w3.weight"], sd[L + "mlp.up_proj.weight"])
    assert torch.equal(params["layers.1.feed_forward.w2.weight"], sd[L + "mlp.down_proj.weight"])
    assert torch.equal(params["layers.1.attention_norm.weight"], sd[L + "input_layernorm.weight"])
    assert torch.equal(params["layers.1.ffn_norm.weight"], sd[L + "post_attention_layernorm.weight"])
    assert torch.equal(params["norm.weight"], sd["model.norm.weight"])
    # RoPE table rebuilt on the host after meta initialisation
    assert model.freqs_cis.device.type == "cpu" and model.freqs_cis.shape == (32, 8)


def test_engine_named_checkpoint_and_dtype_cast(tmp_path):
    """A file in the engine's own key names loads too; fp32 tensors are cast."""
    from src.loader import load_weights
    from src.model import Llama3
    src = Llama3(_args())
    sd = {k: torch.randn(v.shape, generator=torch.Generator().manual_seed(i))
          for i, (k, v) in enumerate(src.state_dict().items())}
    with torch.device("meta"):
        model = Llama3(_args())
    rep = load_weights(model, _save(tmp_path, sd), "cpu", dtype=torch.bfloat16, verbose=False)
    assert rep["missing"] == []
    for k, v in model.state_dict().items():
        assert v.dtype == torch.bfloat16 and torch.equal(v, sd[k].to(torch.bfloat16)), k


def test_missing_and_mismatched_tensors(tmp_path):
    from src.loader import load_weights
    from src.model import Llama3
    sd = _hf_state(1)
    sd.pop("model.layers.0.post_attention_layernorm.weight")
    with torch.device("meta"):
        model = Llama3(_args())
    rep = load_weights(model, _save(tmp_path, sd), "cpu", verbose=False)
    assert rep["missing"] == ["layers.0.ffn_norm.weight"]
    # the missing parameter is materialised (not meta); loaded ones are kept
    assert model.layers[0].ffn_norm.weight.device.type == "cpu"
    assert torch.equal(model.norm.weight, sd["model.norm.weight"])
    sd = _hf_state(2)
    sd["model.norm.weight"] = torch.zeros(TINY["dim"] + 1, dtype=torch.bfloat16)
    with torch.device("meta"):
        model = Llama3(_args())
    with pytest.raises(ValueError, match="Shape mismatch for norm.weight"):
        load_weights(model, _save(tmp_path, sd, "bad.safetensors"), "cpu", verbose=False)
    with pytest.raises(ValueError, match="quantization"):
        load_weights(model, _save(tmp_path, sd, "bad.safetensors"), "cpu", quantization="int4")


def test_w8a16_needs_the_device(tmp_path):
    """The quantiser is a HIP kernel: a host-device W8A16 load fails loudly."""
    from src.loader import build_model_from_weights
    from src.model import Llama3
    with pytest.raises(ValueError, match="requires CUDA"):
        build_model_from_weights(Llama3, _args(), _save(tmp_path, _hf_state(3)), "cpu",
                                 quantization="w8a16")


def test_should_quantize_key():
    from src.quant_utils import get_transformer_linear_names, should_quantize_key
    assert len(get_transformer_linear_names()) == 7
    for mod in get_transformer_linear_names():
        assert should_quantize_key(f"layers.11.{mod}.weight")
        assert not should_quantize_key(f"layers.11.{mod}.scales")
    for key in ("output.weight", "tok_embeddings.weight", "norm.weight", "layers.0.attention_norm.weight",
                "layers.0.ffn_norm.weight", "model.layers.0.self_attn.q_proj.weight", "layers.attention.wq.weight"):
        assert not should_quantize_key(key), key


def test_accuracy_metrics_closed_forms():
    from src import quant_utils as q
    g = torch.Generator().manual_seed(0)
    a = torch.randn(3, 5, 40, generator=g)
    assert abs(float(q.cosine_similarity(a, a)) - 1) < 1e-6
    assert abs(float(q.cosine_similarity(a, -a)) + 1) < 1e-6
    e0, e1 = torch.zeros(2, 8), torch.zeros(2, 8)
    e0[:, 0] = 1
    e1[:, 1] = 3
    assert float(q.cosine_similarity(e0, e1)) == 0.0
    assert q.logits_max_abs_error(a, a + 0.25) == pytest.approx(0.25)
    assert q.logits_relative_error(torch.full((4,), 2.0), torch.full((4,), 3.0)) == pytest.approx(0.5)
    assert q.top1_agreement(a, a) == 1.0
    b = a.clone()
    b[0, 0] = -a[0, 0]                     # row (0, 0)'s argmax moves to its argmin
    assert q.top1_agreement(a, b) == pytest.approx(14 / 15)
    # uniform logits over V classes: perplexity V; a perfect predictor: 1
    V = 37
    labels = torch.randint(0, V, (2, 9), generator=g)
    assert q.perplexity(torch.zeros(2, 9, V), labels) == pytest.approx(V, rel=1e-5)
    sharp = torch.full((9, V), -1e4)
    sharp[torch.arange(8), labels[0, 1:]] = 0.0
    assert q.perplexity(sharp, labels[0]) == pytest.approx(1.0, abs=1e-5)
    ign = labels.clone()
    ign[:, 5:] = -100
    lp = torch.log_softmax(torch.randn(2, 9, V, generator=g), -1)
    ref = math.exp(-float(torch.stack([lp[b, t, ign[b, t + 1]] for b in range(2) for t in range(4)]).mean()))
    assert q.perplexity(lp, ign) == pytest.approx(ref, rel=1e-5)
