"""MI355X (gfx950) attention hot path behind the reference engine's Python API.

Module and function names match Analysis196884/llm-infer-engine's ``src``
package (flash_attn, flash_decode, decode_attn, rope, kv_cache, cuda_graph,
quant_linear, quant_utils, rms_norm, config, model, model_quantized), so model
code written against that API runs on these kernels unchanged.  Every op runs
a hand-written HIP kernel from ``libmiattn.so``; nothing falls back to torch.
"""
