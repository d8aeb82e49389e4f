"""Safetensors checkpoint loader (interface of src/loader.py).

`load_weights(model, path, device, dtype, assign, quantization)` fills an
instantiated (typically meta-device) Llama3 / Llama3Quantized from a
safetensors file in either this engine's key names or Hugging Face Llama
names, with the lm_head tied to the embedding when the file has no
`lm_head.weight` (src/loader.py:8-56).  With quantization="w8a16" the seven
per-layer projections are quantised on the device by mi_quantize_int8, which
is bit-exact with the reference recipe (src/loader.py:59-87,
src/quant_utils.py:7-36).  `build_model_from_weights` is the meta-init +
load + RoPE table entry point (src/loader.py:154-177).

MI355X data path: the file is memory-mapped (safe_open) rather than read
whole into host memory; each tensor is streamed to HBM in 64 MiB pieces
through a ring of pinned host buffers on a copy stream, so the page-in /
memcpy of one piece overlaps the DMA of the previous one, and the host
footprint stays at the ring size instead of the checkpoint size.
Quantisation reads the bf16 master weight where it landed in HBM and writes
int8 + scales next to it.
"""
from __future__ import annotations

import time

import torch

from .quant_utils import quantize_weight_symmetric_per_channel, should_quantize_key

# engine key suffix (below "layers.{i}.") -> Hugging Face Llama suffix
_HF_LAYER_SUFFIX = {
    "attention.wq.weight": "self_attn.q_proj.weight",
    "attention.wk.weight": "self_attn.k_proj.weight",
    "attention.wv.weight": "self_attn.v_proj.weight",
    "attention.wo.weight": "self_attn.o_proj.weight",
    "feed_forward.w1.weight": "mlp.gate_proj.weight",
    "feed_forward.w2.weight": "mlp.down_proj.weight",
    "feed_forward.w3.weight": "mlp.up_proj.weight",
    "attention_norm.weight": "input_layernorm.weight",
    "ffn_norm.weight": "post_attention_layernorm.weight",
}
_HF_TOP = {
    "tok_embeddings.weight": "model.embed_tokens.weight",
    "norm.weight": "model.norm.weight",
    "output.weight": "lm_head.weight",
}
_TIED_SOURCE = "model.embed_tokens.weight"

_CHUNK_BYTES = 64 << 20     # pinned staging piece
_RING = 3                   # staging pieces in flight


def _to_hf_name(model_key: str) -> str:
    """Hugging Face name of an engine state-dict key (unknown keys map to
    themselves), src/loader.py:8-44."""
    if model_key in _HF_TOP:
        return _HF_TOP[model_key]
    if model_key.startswith("layers."):
        _, idx, suffix = model_key.split(".", 2)
        hf = _HF_LAYER_SUFFIX.get(suffix)
        if hf is not None:
            return f"model.layers.{idx}.{hf}"
    return model_key


def _find_source_key(model_key: str, names) -> str | None:
    """Checkpoint key holding `model_key`: the engine name, else the HF name,
    else (lm_head only) the tied embedding; None if absent (src/loader.py:47-56)."""
    for cand in (model_key, _to_hf_name(model_key)):
        if cand in names:
            return cand
    if model_key == "output.weight" and _TIED_SOURCE in names:
        return _TIED_SOURCE
    return None


class _DeviceUploader:
    """Host -> HBM copies through a ring of pinned staging buffers on a side
    stream (default priority).  `upload` returns a device tensor that the
    current stream may use (it waits for the copies)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.stream = torch.cuda.Stream(device=device)
        self.pinned = [torch.empty(_CHUNK_BYTES, dtype=torch.uint8, pin_memory=True)
                       for _ in range(_RING)]
        self.done = [None] * _RING
        self.k = 0

    def upload(self, t: torch.Tensor) -> torch.Tensor:
        t = t.contiguous()
        out = torch.empty(t.shape, dtype=t.dtype, device=self.device)
        n = t.numel() * t.element_size()
        if n == 0:
            return out
        src = t.reshape(-1).view(torch.uint8)
        dst = out.reshape(-1).view(torch.uint8)
        self.stream.wait_stream(torch.cuda.current_stream(self.device))  # `out` is allocated
        for off in range(0, n, _CHUNK_BYTES):
            slot = self.k % _RING
            self.k += 1
            if self.done[slot] is not None:
                self.done[slot].synchronize()        # the piece's previous DMA has drained
            m = min(_CHUNK_BYTES, n - off)
            buf = self.pinned[slot][:m]
            buf.copy_(src[off:off + m])               # page-in + memcpy into pinned memory
            with torch.cuda.stream(self.stream):
                dst[off:off + m].copy_(buf, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(self.stream)
            self.done[slot] = ev
        out.record_stream(self.stream)
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        return out

    def drain(self):
        for ev in self.done:
            if ev is not None:
                ev.synchronize()


def _prepare_weight(model_key, source_tensor, target_shape, device, dtype, quantization):
    """{key: tensor} for one model weight from its checkpoint tensor (already
    on `device`): int8 weight + `.scales` for quantised projections, else the
    tensor cast to `dtype` (src/loader.py:59-87)."""
    if tuple(source_tensor.shape) != tuple(target_shape):
        raise ValueError(f"Shape mismatch for {model_key}: expected {tuple(target_shape)}, "
                         f"got {tuple(source_tensor.shape)}")
    if quantization == "w8a16" and should_quantize_key(model_key):
        qweight, scales = quantize_weight_symmetric_per_channel(source_tensor)
        return {model_key: qweight, model_key[: -len(".weight")] + ".scales": scales.to(dtype=dtype)}
    return {model_key: source_tensor.to(dtype=dtype)}


def _materialize_meta(model: torch.nn.Module, device) -> None:
    """Give parameters / buffers the checkpoint did not provide (still on the
    meta device) uninitialised storage on `device`; loaded ones are kept."""
    for mod in model.modules():
        for name, p in list(mod.named_parameters(recurse=False)):
            if p.device.type == "meta":
                mod.register_parameter(name, torch.nn.Parameter(
                    torch.empty(p.shape, dtype=p.dtype, device=device), requires_grad=p.requires_grad))
        for name, b in list(mod.named_buffers(recurse=False)):
            if b is not None and b.device.type == "meta":
                mod.register_buffer(name, torch.empty(b.shape, dtype=b.dtype, device=device))


def load_weights(model, weights_path, device, dtype=torch.bfloat16, assign=True, quantization=None,
                 verbose=True):
    """Load a safetensors checkpoint into `model` (src/loader.py:90-151).

    Returns {"loaded": n tensors assigned, "missing": model keys that neither
    the file nor the quantiser provided, "unexpected": keys load_state_dict
    did not know}.  Raises ValueError on a shape mismatch and KeyError if
    load_state_dict reports keys missing beyond those.
    """
    from safetensors import safe_open

    if quantization not in (None, "w8a16"):
        raise ValueError(f"unknown quantization {quantization!r} (None or 'w8a16')")
    device = torch.device(device)
    on_gpu = device.type == "cuda"
    torch.cuda.nvtx.range_push("WeightDiskLoad")
    t0 = time.time()
    f = safe_open(str(weights_path), framework="pt", device="cpu")   # memory-mapped
    names = set(f.keys())
    if verbose:
        print(f"    Load: {time.time() - t0:.4f}s ({len(names)} tensors)")
    torch.cuda.nvtx.range_pop()

    torch.cuda.nvtx.range_push("WeightRemapTransfer")
    t1 = time.time()
    uploader = _DeviceUploader(device) if on_gpu else None
    model_dict = model.state_dict()
    remapped = {}
    missing = []
    uploaded = {}   # source key -> device tensor (a tied embedding is read once)
    converted = {}  # source key -> tensor in `dtype`
    for model_key, model_value in model_dict.items():
        if model_key in remapped:
            continue                                   # produced with its weight (scales)
        src = _find_source_key(model_key, names)
        if src is None:
            missing.append(model_key)
            continue
        t = uploaded.get(src)
        if t is None:
            t = f.get_tensor(src)
            if tuple(t.shape) != tuple(model_value.shape):
                raise ValueError(f"Shape mismatch for {model_key}: expected {tuple(model_value.shape)}, "
                                 f"got {tuple(t.shape)}")
            t = uploader.upload(t) if on_gpu else t
            uploaded[src] = t
        prep = _prepare_weight(model_key, t, model_value.shape, device, dtype, quantization)
        if len(prep) == 1:
            # a tensor read for two keys (tied lm_head) is converted once and shared
            prep = {model_key: converted.setdefault(src, prep[model_key])}
        remapped.update(prep)
    del uploaded, converted
    if uploader is not None:
        uploader.drain()
    if verbose:
        print(f"    Transfer: {time.time() - t1:.4f}s ({len(remapped)} tensors)")
    torch.cuda.nvtx.range_pop()

    torch.cuda.nvtx.range_push("WeightStateDictLoad")
    missing = [k for k in missing if k not in remapped]
    result = model.load_state_dict(remapped, strict=False, assign=assign)
    _materialize_meta(model, device)
    model = model.to(device)
    model.eval()
    torch.cuda.nvtx.range_pop()
    unresolved = set(result.missing_keys) - set(missing)
    if unresolved:
        raise KeyError(f"Failed to load required model keys: {sorted(unresolved)}")
    return {"loaded": len(remapped), "missing": sorted(missing),
            "unexpected": sorted(result.unexpected_keys)}


def build_model_from_weights(model_cls, model_args, weights_path, device, dtype=torch.bfloat16,
                             quantization=None):
    """Meta-initialise `model_cls` (Llama3Quantized for quantization="w8a16"),
    load the checkpoint, and rebuild the RoPE table (src/loader.py:154-177).
    Returns (model, report)."""
    from .rope import precompute_freqs_cis

    if quantization == "w8a16":
        from .model_quantized import Llama3Quantized
        model_cls = Llama3Quantized
    torch.cuda.nvtx.range_push("ModelInit")
    with torch.device("meta"):
        model = model_cls(model_args)
    torch.cuda.nvtx.range_pop()
    report = load_weights(model, weights_path, device, dtype=dtype, assign=True,
                          quantization=quantization)
    torch.cuda.nvtx.range_push("FreqsCisPrecompute")
    model.freqs_cis = precompute_freqs_cis(model_args.dim // model_args.n_heads, model_args.max_seq_len,
                                           theta=model_args.rope_theta,
                                           rope_scaling=model_args.rope_scaling)
    model._rope_table = None
    torch.cuda.nvtx.range_pop()
    return model, report
