"""Pins the composed decode-step oracle (oracle/model.py) against an
independent implementation: transformers' LlamaForCausalLM, in fp32 on the CPU.

The engine's module tree is built on the host from the same Hugging Face
checkpoint (src/loader.py, the reference's name remap src/loader.py:8-44), and
oracle.model.decode_step is run token by token from position 0 over a CPU KV
cache -- the reference's decode loop (src/model_quantized.py:42-190,
src/model.py:39-185) one token at a time.  Every position's logits must equal
transformers' full-sequence forward within 1e-4 of the logit scale.  A mistake
in any piece the composition wires together (GQA head map, rotate-half RoPE
convention or llama3 scaling, SwiGLU roles, residual order, the final norm, a
tied head) moves logits by far more than that.

The W8A16 case quantises the seven per-layer projections with the oracle's
quantiser and gives transformers the dequantised weights q * s (the reference
test's own reference, tests/quant_unit.py:64-77), activations in fp32.
"""
import pytest
import torch

from oracle import model as omodel
from oracle import quant as oq

SHAPE = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, hidden_dim=160)
LLAMA3_ROPE = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
               "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
SEQ = 14
T = 32
_HF_LINEARS = {"attention.wq": "self_attn.q_proj", "attention.wk": "self_attn.k_proj",
               "attention.wv": "self_attn.v_proj", "attention.wo": "self_attn.o_proj",
               "feed_forward.w1": "mlp.gate_proj", "feed_forward.w2": "mlp.down_proj",
               "feed_forward.w3": "mlp.up_proj"}


def _hf_model(tied, rope_scaling, seed):
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
            if "norm" in name:             # all-ones at init: perturb so the weights matter
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif "proj" in name:           # larger than init so attention is far from uniform
                p.mul_(3.0)
            p.copy_(p.to(torch.bfloat16).float())
    return m


def _engine_from(hf, tied, rope_scaling, tmp_path):
    from safetensors.torch import save_file

    from src.config import ModelArgs
    from src.loader import build_model_from_weights
    from src.model import Llama3
    sd = {k: v.detach().contiguous().clone() for k, v in hf.state_dict().items() if "rotary" not in k}
    if tied:
        sd.pop("lm_head.weight", None)
    path = tmp_path / "model.safetensors"
    save_file(sd, str(path))
    args = ModelArgs(max_batch_size=2, max_seq_len=T, device="cpu", rope_scaling=rope_scaling, **SHAPE)
    model, rep = build_model_from_weights(Llama3, args, path, "cpu", dtype=torch.float32)
    assert rep["missing"] == [] and rep["unexpected"] == []
    return model, args


class _Q(torch.nn.Module):
    """A W8A16Linear's parameters as the oracle reads them (int8 weight, scales)."""

    def __init__(self, q, s):
        super().__init__()
        self.register_buffer("weight", q)
        self.register_buffer("scales", s)


def _quantise(model, hf):
    """Replace each per-layer projection of the engine tree with int8 + bf16-valued
    scales (oracle quantiser) and give transformers the dequantised q * s."""
    hf_params = dict(hf.named_parameters())
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            for name, hf_name in _HF_LINEARS.items():
                parent, attr = name.split(".")
                lin = getattr(getattr(layer, parent), attr)
                q, s = oq.quantize_per_channel(lin.weight.float().numpy(), "bfloat16")
                q, s = torch.from_numpy(q), torch.from_numpy(s)
                assert int(q.abs().max()) <= 127
                setattr(getattr(layer, parent), attr, _Q(q, s))
                hf_params[f"model.layers.{i}.{hf_name}.weight"].copy_(q.float() * s)


def _decode_all(model, args, tokens):
    B = tokens.shape[0]
    D = args.dim // args.n_heads
    ck = torch.zeros(args.n_layers, args.max_batch_size, args.n_kv_heads, T, D)
    cv = torch.zeros_like(ck)
    out = [omodel.decode_step(model, tokens[:, t:t + 1], t, ck, cv, args.norm_eps)
           for t in range(tokens.shape[1])]
    return torch.cat(out, 1).reshape(B, tokens.shape[1], -1), ck, cv


@pytest.mark.parametrize("w8a16", [False, True])
@pytest.mark.parametrize("tied,rope_scaling", [(False, None), (True, LLAMA3_ROPE)])
def test_decode_step_matches_transformers(tmp_path, tied, rope_scaling, w8a16):
    hf = _hf_model(tied, rope_scaling, seed=11 + int(w8a16))
    model, args = _engine_from(hf, tied, rope_scaling, tmp_path)
    if w8a16:
        _quantise(model, hf)
    tokens = torch.randint(0, SHAPE["vocab_size"], (2, SEQ), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = hf(tokens).logits.float()
    got, ck, cv = _decode_all(model, args, tokens)
    scale = float(ref.abs().max())
    err = float((got - ref).abs().max())
    assert err < 1e-4 * scale, (err, scale)
    assert torch.equal(got.argmax(-1), ref.argmax(-1))
    # slots past the last decoded position are never written
    assert not ck[:, :, :, SEQ:].any() and not cv[:, :, :, SEQ:].any()


_MISTAKES = {
    # the sin sign flipped (rotation by -theta)
    "rope_sign": lambda m: m.setattr(omodel.orope, "rotate",
                                     (lambda r: lambda x, c, s: r(x, c, -s))(omodel.orope.rotate)),
    # query heads grouped as h % Hkv instead of h // G
    "gqa_map": lambda m: m.setattr(omodel.ora, "decode", (lambda d: lambda q, k, v, **kw: (
        lambda o: (o[0][:, _inv_perm(q.shape[1], k.shape[1])], o[1]))(
        d(q[:, _perm(q.shape[1], k.shape[1])], k, v, **kw)))(omodel.ora.decode)),
    # RMSNorm without its weight
    "norm_weight": lambda m: m.setattr(omodel.oq, "rmsnorm", (lambda r: lambda x, w, eps: r(
        x, torch.ones_like(w), eps))(omodel.oq.rmsnorm)),
}


def _perm(hq, hkv):
    """Row order that puts query head h in kv group h % Hkv when grouped by h // G."""
    g = hq // hkv
    return [j * hkv + i for i in range(hkv) for j in range(g)]


def _inv_perm(hq, hkv):
    p = _perm(hq, hkv)
    inv = [0] * hq
    for i, j in enumerate(p):
        inv[j] = i
    return inv


@pytest.mark.parametrize("mistake", sorted(_MISTAKES))
def test_bar_fails_planted_oracle_mistakes(tmp_path, monkeypatch, mistake):
    """The same comparison fails when a plausible mistake is planted in the
    oracle (on the CPU): the 1e-4 bar is not satisfied by a wrong composition."""
    hf = _hf_model(False, None, seed=11)
    model, args = _engine_from(hf, False, None, tmp_path)
    tokens = torch.randint(0, SHAPE["vocab_size"], (2, SEQ), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = hf(tokens).logits.float()
    _MISTAKES[mistake](monkeypatch)
    got, _, _ = _decode_all(model, args, tokens)
    assert float((got - ref).abs().max()) > 1e-2 * float(ref.abs().max())
