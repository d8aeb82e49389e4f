"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain fp32 torch (CPU) and numpy, the arithmetic of
the reference engine's attention path (Analysis196884/llm-infer-engine,
``src/*.py``), each function citing the reference lines it follows.  It is the
checker the HIP kernels are compared against, and the CPU baseline timed by
``bench.py``.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product package never does.

How each part is pinned (see tests/test_oracle_*.py):
  attention.prefill   SDPA (the routine the reference's own test uses,
                      src/flash_attn.py:128-129), brute-force loops, row-0 and
                      constant-key closed forms, MHA reduction.
  attention.decode    SDPA with a boolean mask, L=1 and all-masked closed forms,
                      mask/seq_lens equivalences.
  attention.split_*   split invariance: combine(partials) == single pass.
  rope                float64 cos/sin of the published angle formula,
                      identity at position 0, norm preservation, relative-
                      position invariance, piecewise llama3 scaling rules.
  kv                  slot formula vs torch's own contiguous indexing.
  quant               hand-built rows (zeros, ties, +-amax), |q| <= 127.
  linear              integer-exact cases computed with Python ints.
  norm                constant-row closed form.
  model               transformers' LlamaForCausalLM (fp32, CPU) on the same
                      checkpoint, token by token: logits within 1e-4 of scale,
                      bf16 and W8A16 weights, default and llama3 RoPE, tied and
                      untied heads; planted mistakes fail that bar.
"""
