"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (`value`): BASELINE config 2 — causal GQA prefill, bf16, B4 S2048
32/8 heads D64, fp32 LSE output, in TFLOP/s of algorithmic work
(4*B*Hq*S^2*D/2 = 68.72 GFLOP per step).  The same line carries, under
`extra`, the HBM-bound decode configs (3: B16 24/8 D128 T8192 ragged lengths;
4: B1 L=131072, split sweep) in GB/s, the W8A16 decode step (config 5) in
tokens/s, and the W8A16 prefill GEMM (one layer's projections at config 2's
8192 tokens) in TFLOP/s, each with its own roofline; config 1 and config 2's
attention block in the model layout (RoPE(K) + KV append + attention with q's
RoPE fused) in TFLOP/s; and the CPU baseline (the fp32 oracle on the host
cores, one bounded sample per config, under each leg).

A step is one flash_attention call on resident inputs.  Timing: untimed
warm-up (at least W steps and at least 0.25 s of back-to-back steps, so the GPU
clock has settled), then K steps between torch.cuda.synchronize() calls, with
HIP events (torch's current stream — the stream the kernels are launched on).
Decode calls are replayed from a captured hipGraph holding one call per
rotating buffer set (consecutive calls in one graph, like a captured decode
loop; the sets are large enough that the 256 MB MALL cannot serve re-reads).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "llm-infer-engine_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA, TFLOP/s


def _cpu_name() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _traffic(summary: str, key: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary under profiles/ (a `key: bytes` line), or None."""
    f = ROOT / "profiles" / summary
    try:
        for ln in f.read_text().splitlines():
            if ln.startswith(key + ":"):
                return int(ln.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def _settle(torch, fn, warmup: int, min_s: float = 0.25) -> None:
    """Untimed warm-up: at least `warmup` calls and at least `min_s` seconds of
    back-to-back work, so the GPU clock has settled before the timed region
    (a handful of sub-millisecond launches does not get there)."""
    import time
    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < min_s:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def bench_prefill(torch, steps: int, warmup: int) -> dict:
    from src.flash_attn import flash_attention
    dev = torch.device("cuda:0")
    B, Hq, Hkv, S, D = 4, 32, 8, 2048, 64
    g = torch.Generator("cpu").manual_seed(0)
    # config 2: Q/K/V ~ N(0,1), Q scaled by 1/sqrt(64) (softmax scale folded in)
    q = (torch.randn((B, Hq, S, D), generator=g) / 8.0).to(torch.bfloat16).to(dev)
    k = torch.randn((B, Hkv, S, D), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((B, Hkv, S, D), generator=g).to(torch.bfloat16).to(dev)
    flops = 4.0 * B * Hq * S * S * D / 2
    step = lambda: flash_attention(q, k, v, sm_scale=1.0, return_lse=True)  # noqa: E731
    _settle(torch, step, warmup)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    # A step is exactly one kernel launch (prefill_sp_kernel) on torch's current
    # stream, so the timed region's average is the kernel's average launch
    # duration (back-to-back launches, no host gaps).
    achieved = flops / (ms * 1e-3) / 1e12
    return {
        "ms_per_step": ms,
        "value": achieved,
        "kernel_ms": ms,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                     "traffic": _traffic("prefill_config2_traffic.md", "hbm_bytes_per_launch")},
        "flops": flops,
    }


def _graph_decode(torch, fn, n_sets):
    """One hipGraph holding n_sets consecutive decode calls, one per rotating
    buffer set (a captured decode loop: consecutive calls share one launch)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_sets):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for i in range(n_sets):
            fn(i)
    return gr


def _time_graph(torch, graph, calls, steps, warmup):
    """ms per call: replays of `graph` (holding `calls` calls) covering at
    least `steps` calls, after a settled warm-up."""
    replays = max(1, -(-steps // calls))
    _settle(torch, graph.replay, max(1, -(-warmup // calls)))
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(replays):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / (replays * calls)


def bench_decode_cfg3(torch, steps: int, warmup: int) -> dict:
    from src.flash_decode import flash_decode
    dev = torch.device("cuda:0")
    g = torch.Generator("cpu").manual_seed(0)
    lens = torch.randint(1024, 8193, (16,), generator=g)
    n_sets = 3  # 3 x 537 MB of K/V: well past the 256 MB MALL
    qs, ks, vs = [], [], []
    for _ in range(n_sets):
        qs.append(torch.randn((16, 24, 1, 128), generator=g).to(torch.bfloat16).to(dev))
        ks.append(torch.randn((16, 8, 8192, 128), generator=g).to(torch.bfloat16).to(dev))
        vs.append(torch.randn((16, 8, 8192, 128), generator=g).to(torch.bfloat16).to(dev))
    sl = lens.to(dev)
    nbytes = int(lens.sum()) * 8 * 128 * 2 * 2 + 2 * 16 * 24 * 128 * 2
    graph = _graph_decode(torch, lambda i: flash_decode(qs[i], ks[i], vs[i], seq_lens=sl), n_sets)
    ms = _time_graph(torch, graph, n_sets, max(steps, 21), warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del graph
    # the reference API's call (src/model.py:83): the same keys through a bool mask
    mask = (torch.arange(8192)[None, :] < lens[:, None]).to(dev)
    graph = _graph_decode(torch, lambda i: flash_decode(qs[i], ks[i], vs[i], mask=mask), n_sets)
    ms_m = _time_graph(torch, graph, n_sets, max(steps, 21), warmup)
    gbs_m = nbytes / (ms_m * 1e-3) / 1e9
    out = {
        "config": "3: decode B16 24/8 D128 T8192 L~U[1024,8192] (sum 96634), seq_lens, hipGraph",
        "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": ms, "bytes": nbytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": _traffic("decode_config3_4_traffic.md",
                                         "hbm_bytes_per_launch_config3")},
        "mask_path": {"call": "flash_decode(q, k, v, mask=[16, 8192] bool = arange < L_b)",
                      "value": round(gbs_m, 1), "unit": "GB/s", "ms_per_step": ms_m,
                      "of_seq_lens_path": round(gbs_m / gbs, 3)},
    }
    del graph, ks, vs
    torch.cuda.empty_cache()
    return out


def bench_decode_cfg4(torch, steps: int, warmup: int) -> dict:
    from src.flash_decode import flash_decode
    dev = torch.device("cuda:0")
    g = torch.Generator("cpu").manual_seed(0)
    n_sets = 2  # 2 x 537 MB
    qs = [torch.randn((1, 24, 1, 128), generator=g).to(torch.bfloat16).to(dev) for _ in range(n_sets)]
    ks = [torch.randn((1, 8, 131072, 128), generator=g).to(torch.bfloat16).to(dev) for _ in range(n_sets)]
    vs = [torch.randn((1, 8, 131072, 128), generator=g).to(torch.bfloat16).to(dev) for _ in range(n_sets)]
    nbytes = 131072 * 8 * 128 * 2 * 2 + 2 * 24 * 128 * 2
    from src import _lib
    sweep, ranges = {}, {}
    for splits in (16, 32, 64, 128):
        # the key ranges the library runs for this request (too few splits to
        # fill the CUs are subdivided: 16 requested -> 32 ranges here)
        ranges[str(splits)] = int(_lib.load().mi_decode_effective_splits(1, 24, 8, 131072, 128,
                                                                         splits))
        graph = _graph_decode(
            torch, lambda i, s=splits: flash_decode(qs[i], ks[i], vs[i], num_splits=s), n_sets)
        ms = _time_graph(torch, graph, n_sets, max(steps, 20), warmup)
        sweep[str(splits)] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        del graph
    best = max(sweep.values())
    out = {"config": "4: decode B1 L131072 24/8 D128, splits sweep (combine included)",
           "unit": "GB/s", "by_splits": sweep, "value": best,
           "key_ranges_by_splits": ranges,
           "roofline": {"bound": "hbm", "achieved": best, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(best / HBM_PEAK_GBS, 4),
                        "traffic": _traffic("decode_config3_4_traffic.md",
                                            "hbm_bytes_per_launch_config4")}}
    del ks, vs
    torch.cuda.empty_cache()
    return out


def bench_config5(torch, steps: int, warmup: int) -> dict:
    """Llama-3.2-1B W8A16 decode step, B8, context 4096, hipGraph replay."""
    from src.config import ModelArgs
    from src.cuda_graph import CUDAGraphDecodeRunner
    from src.kv_cache import KVCache
    from src.model_quantized import build_random_quantized
    dev = torch.device("cuda:0")
    args = ModelArgs(max_batch_size=8, max_seq_len=8192, device=str(dev))
    model = build_random_quantized(args, seed=0, device=str(dev))
    kv = KVCache(args, dtype=torch.bfloat16)
    runner = CUDAGraphDecodeRunner(model, args, kv, str(dev), batch_size=8)
    g = torch.Generator(device=dev).manual_seed(0)
    kv.k[:, :, :, :4096].normal_(generator=g)
    kv.v[:, :, :, :4096].normal_(generator=g)
    tok = torch.randint(0, args.vocab_size, (8, 1), generator=torch.Generator().manual_seed(0)).to(dev)
    runner.set_inputs(tok, 4096)
    ms = _time_graph(torch, runner.graph, 1, max(steps, 20), warmup)
    # int8 linears + bf16 lm_head + K/V read (4097 slots) + scales, per step
    D, L = 64, 16
    lin = L * (2048 * 2048 * 2 + 2 * 512 * 2048 + 3 * 2048 * 8192)
    nbytes = lin + L * (2048 * 2 + 512 * 2 + 8192 * 3) * 2 + 128256 * 2048 * 2 \
        + L * 8 * 8 * 4097 * D * 2 * 2
    out = {"config": "5: Llama-3.2-1B random-init W8A16 decode step, B8, ctx 4096, hipGraph",
           "value": round(8 / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": ms,
           "bytes": nbytes,
           "roofline": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "traffic": _traffic("decode_step_config5_traffic.md",
                                            "hbm_bytes_per_step")}}
    del runner, model, kv
    torch.cuda.empty_cache()
    return out


def bench_w8a16_prefill(torch, steps: int, warmup: int) -> dict:
    """The seven W8A16 projections of one Llama-3.2-1B layer at config 2's token
    count (M = 4 x 2048), back to back, through the model's GEMM dispatch: wq,
    wk and wv in one mi_w8a16_gemm_multi launch (QuantizedAttention.qkv), w1 and
    w3 with the SwiGLU gating in one mi_w8a16_gemm_swiglu launch
    (QuantizedFeedForward), wo and w2 with the block's residual add in their
    epilogue (w8a16_gemm_residual).  per_projection also times each projection
    on its own (w8a16_gemm_mfma, the split-K form where the tile grid leaves
    CUs idle)."""
    from src import _lib
    from src.quant_linear import (gemm_multi_worth, swiglu_worth, w8a16_gemm_mfma,
                                  w8a16_gemm_multi, w8a16_gemm_residual, w8a16_gemm_swiglu)
    dev = torch.device("cuda:0")
    _lib.load()
    M = 4 * 2048
    shapes = [("wq", 2048, 2048), ("wk", 512, 2048), ("wv", 512, 2048), ("wo", 2048, 2048),
              ("w1", 8192, 2048), ("w3", 8192, 2048), ("w2", 2048, 8192)]   # (name, N, K)
    g = torch.Generator("cpu").manual_seed(0)
    xs = {K: torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev) for K in (2048, 8192)}
    ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev) for _, N, K in shapes]
    ss = [(torch.rand(N, generator=g) * 0.02 + 1e-3).to(torch.bfloat16).to(dev) for _, N, _ in shapes]

    def call(i):
        _, N, K = shapes[i]
        w8a16_gemm_mfma(xs[K], ws[i], ss[i])

    fuse_qkv = gemm_multi_worth(M, 2048, [N for _, N, _ in shapes[:3]], dev)

    def qkv():
        if fuse_qkv:
            w8a16_gemm_multi(xs[2048], [(ws[i], ss[i]) for i in range(3)])
        else:
            for i in range(3):
                call(i)

    fuse_ffn = swiglu_worth(M, 2048, 8192, dev)

    def ffn_chain():   # the op chain of src/model.py:23
        torch.nn.functional.silu(w8a16_gemm_mfma(xs[2048], ws[4], ss[4])) * \
            w8a16_gemm_mfma(xs[2048], ws[5], ss[5])

    def ffn_in():
        if fuse_ffn:
            w8a16_gemm_swiglu(xs[2048], ws[4], ss[4], ws[5], ss[5])
        else:
            ffn_chain()

    res = torch.randn(M, 2048, generator=g).to(torch.bfloat16).to(dev)

    def call_res(i):
        _, N, K = shapes[i]
        w8a16_gemm_residual(xs[K], ws[i], ss[i], res)

    def step():
        qkv()
        call_res(3)
        ffn_in()
        call_res(6)

    def timed(fn, n):
        _settle(torch, fn, warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    ms = timed(step, steps)
    flops = sum(2.0 * M * N * K for _, N, K in shapes)
    per = {}
    for i, (name, N, K) in enumerate(shapes):
        t = timed(lambda: call(i), steps)
        per[name] = {"N": N, "K": K, "us": round(t * 1e3, 2),
                     "tflops": round(2.0 * M * N * K / (t * 1e-3) / 1e12, 1)}
    t = timed(qkv, steps)
    per["wq+wk+wv"] = {"N": 3072, "K": 2048, "us": round(t * 1e3, 2), "one_launch": fuse_qkv,
                       "tflops": round(2.0 * M * 3072 * 2048 / (t * 1e-3) / 1e12, 1)}
    t = timed(ffn_in, steps)
    per["silu(w1)*w3"] = {"N": 16384, "K": 2048, "us": round(t * 1e3, 2), "one_launch": fuse_ffn,
                          "tflops": round(2.0 * M * 16384 * 2048 / (t * 1e-3) / 1e12, 1)}
    t = timed(ffn_chain, steps)
    per["silu(w1)*w3 as separate ops"] = {"us": round(t * 1e3, 2)}
    for i, name in ((3, "wo+residual"), (6, "w2+residual")):
        per[name] = {"us": round(timed(lambda: call_res(i), steps) * 1e3, 2)}
    tf = flops / (ms * 1e-3) / 1e12
    # the dominant shape (w1/w3: 2 of the 7 calls, 54 % of the flops)
    dom = per["w1"]
    out = {"config": "W8A16 prefill projections of one Llama-3.2-1B layer as the model runs "
                     "them (wq|wk|wv one launch, silu(w1)*w3 one launch, wo and w2 with the residual "
                     "add in the epilogue), M = 8192 "
                     "tokens (config 2's B4 x S2048), bf16 activations, int8 weights, bf16 scales",
           "value": round(tf, 1), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "flops_per_step": flops, "per_projection": per,
           "roofline": {"bound": "mfma", "kernel": "w8a16_gemm_kernel (w1 shape)",
                        "achieved": dom["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(dom["tflops"] / BF16_PEAK_TFLOPS, 4),
                        "traffic": _traffic("w8a16_gemm_traffic.md", "hbm_bytes_per_launch_w1")}}
    del xs, ws, ss, res
    torch.cuda.empty_cache()
    return out


def bench_loader(torch) -> dict:
    """Checkpoint load of a Llama-3.2-1B-shaped Hugging Face safetensors file
    (random bf16 values, tied embeddings, 2.47 GB) written to a temporary
    directory: build_model_from_weights for bf16 and for W8A16 (on-device
    quantisation).  The file was just written, so it is served from the page
    cache: the figure is memcpy + host->HBM DMA + quantisation, not disk."""
    import contextlib
    import tempfile
    from safetensors.torch import save_file
    from src.config import ModelArgs
    from src.loader import build_model_from_weights
    from src.model import Llama3
    dev = torch.device("cuda:0")
    args = ModelArgs(max_seq_len=256, device=str(dev))
    d, hd, kv = args.dim, args.hidden_dim, args.n_kv_heads * (args.dim // args.n_heads)
    shapes = {"model.embed_tokens.weight": (args.vocab_size, d), "model.norm.weight": (d,)}
    for i in range(args.n_layers):
        p = f"model.layers.{i}."
        shapes.update({p + "self_attn.q_proj.weight": (d, d), p + "self_attn.k_proj.weight": (kv, d),
                       p + "self_attn.v_proj.weight": (kv, d), p + "self_attn.o_proj.weight": (d, d),
                       p + "mlp.gate_proj.weight": (hd, d), p + "mlp.up_proj.weight": (hd, d),
                       p + "mlp.down_proj.weight": (d, hd), p + "input_layernorm.weight": (d,),
                       p + "post_attention_layernorm.weight": (d,)})
    g = torch.Generator("cpu").manual_seed(0)
    sd = {k: (torch.randn(s, generator=g) * 0.02).to(torch.bfloat16) for k, s in shapes.items()}
    nbytes = sum(v.numel() * 2 for v in sd.values())
    out = {"config": "Llama-3.2-1B-shaped HF safetensors, tied embeddings, random bf16, page-cached",
           "bytes": nbytes, "unit": "GB/s"}
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        path = os.path.join(tmp, "model.safetensors")
        save_file(sd, path)
        del sd
        # the first load also pays one-time set-up (pinned staging buffers, the
        # allocator's first HBM reservations, page-table population of the
        # mapping): reported apart from the steady-state loads that follow
        for label, quant in (("first_load_w8a16", "w8a16"), ("bf16", None), ("w8a16", "w8a16")):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with contextlib.redirect_stdout(sys.stderr):   # the loader's progress lines
                model, _ = build_model_from_weights(Llama3, args, path, str(dev),
                                                    dtype=torch.bfloat16, quantization=quant)
            torch.cuda.synchronize()
            t = time.perf_counter() - t0
            out[label] = {"seconds": round(t, 3), "GB_per_s": round(nbytes / t / 1e9, 2)}
            del model
    out["value"] = out["w8a16"]["GB_per_s"]
    return out


def _cpu_threads(torch) -> dict:
    """Use every CPU this process may run on (the lease's share of the host,
    from the affinity mask) and record what the host offers."""
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    torch.set_num_threads(aff)
    return {"cpu": _cpu_name(), "os_cpu_count": os.cpu_count(), "affinity_cpus": aff,
            "torch_threads": torch.get_num_threads()}


def _cpu_median(fn, warm: int = 2, reps: int = 5) -> float:
    """Median wall time of `reps` calls after `warm` untimed ones."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def _cpu_entry(value, unit, host, sample, t) -> dict:
    return {"value": value, "unit": unit, "cores": host["torch_threads"], "kind": "port",
            "sample": f"{sample}; median of 5 after 2 warm-ups: {t:.3f} s per call",
            "host": host}


def cpu_baselines(torch) -> dict:
    """The fp32 CPU oracle (this build's restatement of the reference maths,
    oracle/) on the host cores, one bounded sample per BASELINE config, each
    scaled to that config's metric.  Inputs are bf16-rounded like the GPU legs'."""
    from oracle import attention as ora
    from oracle import quant as oq
    from oracle import rope as orope
    host = _cpu_threads(torch)
    out = {}
    g = torch.Generator("cpu").manual_seed(0)

    # config 1: fp32 RoPE (theta 5e5) on Q and K + causal GQA prefill, B1 S512 32/8 D64
    q = torch.randn((1, 32, 512, 64), generator=g)
    k = torch.randn((1, 8, 512, 64), generator=g)
    v = torch.randn((1, 8, 512, 64), generator=g)
    cos, sin = orope.cos_sin(orope.freqs_cis(64, 512, 500000.0), torch.float32)
    fl1 = 4.0 * 32 * 512 * 512 * 64 / 2
    t = _cpu_median(lambda: ora.prefill(orope.rotate(q, cos, sin), orope.rotate(k, cos, sin), v))
    out["config1"] = _cpu_entry(round(fl1 / t / 1e12, 5), "TFLOP/s", host,
                                "config 1 whole (RoPE on Q/K + prefill, 1.074 GFLOP)", t)

    # config 2: the whole step (B4 S2048 32/8 D64, fp32 LSE)
    q = (torch.randn((4, 32, 2048, 64), generator=g) / 8.0).to(torch.bfloat16)
    k = torch.randn((4, 8, 2048, 64), generator=g).to(torch.bfloat16)
    v = torch.randn((4, 8, 2048, 64), generator=g).to(torch.bfloat16)
    fl2 = 4.0 * 4 * 32 * 2048 * 2048 * 64 / 2
    t = _cpu_median(lambda: ora.prefill(q, k, v, sm_scale=1.0))
    out["config2"] = _cpu_entry(round(fl2 / t / 1e12, 4), "TFLOP/s", host,
                                "config 2 whole step (68.72 GFLOP)", t)
    del q, k, v

    # config 3: the first 4 of the 16 sequences (their own lengths), bf16 K/V
    g3 = torch.Generator("cpu").manual_seed(0)
    lens = torch.randint(1024, 8193, (16,), generator=g3)[:4]
    Lm = int(lens.max())
    q = torch.randn((4, 24, 1, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((4, 8, Lm, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((4, 8, Lm, 128), generator=g).to(torch.bfloat16)
    by3 = int(lens.sum()) * 8 * 128 * 2 * 2 + 2 * 4 * 24 * 128 * 2
    t = _cpu_median(lambda: ora.decode(q, k, v, seq_lens=lens))
    out["config3"] = _cpu_entry(round(by3 / t / 1e9, 2), "GB/s", host,
                                f"config 3, sequences 0-3 (lengths {lens.tolist()}, "
                                f"{by3 / 1e6:.1f} MB of bf16 K/V + q/o)", t)
    del q, k, v

    # config 4: a quarter of the context (32768 of 131072 keys)
    q = torch.randn((1, 24, 1, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 8, 32768, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 8, 32768, 128), generator=g).to(torch.bfloat16)
    by4 = 32768 * 8 * 128 * 2 * 2 + 2 * 24 * 128 * 2
    t = _cpu_median(lambda: ora.decode(q, k, v))
    out["config4"] = _cpu_entry(round(by4 / t / 1e9, 2), "GB/s", host,
                                f"config 4 at 32768 of 131072 keys ({by4 / 1e6:.1f} MB)", t)
    del q, k, v

    # config 5: one of the 16 W8A16 layers (int8 weights dequantised q*s inside
    # every call) and 1/16 of the bf16 lm_head rows; step = 16 x (layer + slice)
    dim, hid, Hq, Hkv, D, B, pos = 2048, 8192, 32, 8, 64, 8, 4096

    def w8(n, kk):
        return (torch.randint(-127, 128, (n, kk), generator=g, dtype=torch.int8),
                (torch.rand((n, 1), generator=g) * 2e-3 + 1e-3).to(torch.bfloat16))
    wq, wk, wv, wo = w8(Hq * D, dim), w8(Hkv * D, dim), w8(Hkv * D, dim), w8(dim, Hq * D)
    w1, w3, w2 = w8(hid, dim), w8(hid, dim), w8(dim, hid)
    nw1 = torch.ones(dim, dtype=torch.bfloat16)
    ck = torch.randn((B, Hkv, pos + 1, D), generator=g).to(torch.bfloat16)
    cv = torch.randn((B, Hkv, pos + 1, D), generator=g).to(torch.bfloat16)
    h0 = torch.randn((B, 1, dim), generator=g).to(torch.bfloat16)
    lm = (torch.randn((128256 // 16, dim), generator=g) * 0.02).to(torch.bfloat16)
    cs, sn = orope.cos_sin(orope.freqs_cis(D, pos + 1, 500000.0)[pos:pos + 1], torch.bfloat16)

    def layer():
        x = oq.rmsnorm(h0, nw1, 1e-5)
        xq = oq.w8a16(x, *wq).view(B, 1, Hq, D).transpose(1, 2)
        xk = oq.w8a16(x, *wk).view(B, 1, Hkv, D).transpose(1, 2)
        xv = oq.w8a16(x, *wv).view(B, 1, Hkv, D).transpose(1, 2)
        xq = orope.rotate(xq, cs, sn)
        ck[:, :, pos] = orope.rotate(xk, cs, sn)[:, :, 0]
        cv[:, :, pos] = xv[:, :, 0]
        o, _ = ora.decode(xq, ck, cv)
        h = (h0.float() + oq.w8a16(o.to(torch.bfloat16).transpose(1, 2).reshape(B, 1, dim),
                                   *wo).float()).to(torch.bfloat16)
        x = oq.rmsnorm(h, nw1, 1e-5)
        a = oq.w8a16(x, *w1).float()
        gg = (a * torch.sigmoid(a)).to(torch.bfloat16).float() * oq.w8a16(x, *w3).float()
        return (h.float() + oq.w8a16(gg.to(torch.bfloat16), *w2).float()).to(torch.bfloat16)

    def head():
        x = oq.rmsnorm(h0, nw1, 1e-5)
        return x.float() @ lm.float().t()
    t_l = _cpu_median(layer)
    t_h = _cpu_median(head)
    t5 = 16 * (t_l + t_h)
    out["config5"] = _cpu_entry(round(B / t5, 2), "tokens/s", host,
                                f"config 5 from one W8A16 layer ({t_l:.3f} s, int8 -> fp32 "
                                f"dequantisation inside) and 1/16 of the lm_head rows "
                                f"({t_h:.3f} s), step = 16 x (layer + slice) = {t5:.2f} s", t_l)
    return out


def bench_prefill_d128(torch, steps: int, warmup: int) -> dict:
    """Causal GQA prefill at the Llama-3.2-3B head shape of configs 3 and 4
    (B4 S2048 24/8 heads D128, bf16, fp32 LSE): prefill_sp2_kernel<bf16,128>,
    one launch per step, timed as the headline leg is."""
    from src.flash_attn import flash_attention
    dev = torch.device("cuda:0")
    B, Hq, Hkv, S, D = 4, 24, 8, 2048, 128
    g = torch.Generator("cpu").manual_seed(1)
    q = torch.randn((B, Hq, S, D), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((B, Hkv, S, D), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((B, Hkv, S, D), generator=g).to(torch.bfloat16).to(dev)
    flops = 4.0 * B * Hq * S * S * D / 2
    step = lambda: flash_attention(q, k, v, return_lse=True)  # noqa: E731
    _settle(torch, step, warmup)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    achieved = flops / (ms * 1e-3) / 1e12
    return {"config": "causal GQA prefill B4 S2048 Hq24 Hkv8 D128 (the 3B head shape of configs "
                      "3/4), bf16, fp32 LSE",
            "value": round(achieved, 1), "unit": "TFLOP/s", "ms_per_step": ms, "flops": flops,
            "roofline": {"bound": "mfma", "kernel": "prefill_sp2_kernel<bf16,128>",
                         "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                         "traffic": _traffic("prefill_d128_traffic.md", "hbm_bytes_per_launch")}}


def bench_w8a16_prefill_e2e(torch, steps: int, warmup: int) -> dict:
    """The reference's timed prefill (main.py:233-243): the whole Llama-3.2-1B
    random-init W8A16 model over a prompt, model(tokens, start_pos=0,
    kv_cache=...), logits of the last position.  Batch 4 x 2048 tokens
    (config 2's token count).  Work per call: the seven int8 projections of 16
    layers (2 FLOP per weight and token), causal attention (4*B*Hq*S^2*D/2 per
    layer) and the last rows' lm_head."""
    from src.config import ModelArgs
    from src.kv_cache import KVCache
    from src.model_quantized import build_random_quantized
    dev = torch.device("cuda:0")
    B, S = 4, 2048
    args = ModelArgs(max_batch_size=B, max_seq_len=S, device=str(dev))
    model = build_random_quantized(args, seed=0, device=str(dev))
    kv = KVCache(args, dtype=torch.bfloat16)
    tokens = torch.randint(0, args.vocab_size, (B, S),
                           generator=torch.Generator().manual_seed(0)).to(dev)
    hd = args.dim // args.n_heads
    kvd = args.n_kv_heads * hd
    ffn = 8192
    lin_params = args.n_layers * (2 * args.dim * args.dim + 2 * kvd * args.dim
                                  + 3 * ffn * args.dim)
    flops = (2.0 * B * S * lin_params
             + args.n_layers * 4.0 * B * args.n_heads * S * S * hd / 2
             + 2.0 * B * args.vocab_size * args.dim)

    def step():
        with torch.no_grad():
            return model(tokens, start_pos=0, kv_cache=kv)
    _settle(torch, step, max(2, warmup // 4), min_s=0.5)
    n = max(5, steps // 2)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(n):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / n
    out = {"config": "Llama-3.2-1B random-init W8A16 prefill, B4 x 2048 tokens, "
                     "model(tokens, start_pos=0, kv_cache) (logits of the last position)",
           "value": round(flops / (ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s",
           "ms_per_step": ms, "tokens_per_s": round(B * S / (ms * 1e-3), 1), "flops": flops,
           "steps": n}
    del model, kv
    torch.cuda.empty_cache()
    return out


def bench_prefill_cfg1(torch, steps: int, warmup: int) -> dict:
    """Config 1 on the GPU (fp32 RoPE on Q and K + causal GQA prefill, B1 S512
    32/8 D64): the parity configuration, timed beside its CPU baseline."""
    from src.flash_attn import flash_attention
    from src.rope import apply_rotary, build_rope_cos_sin, precompute_freqs_cis
    dev = torch.device("cuda:0")
    g = torch.Generator("cpu").manual_seed(0)
    q = torch.randn((1, 32, 512, 64), generator=g).to(dev)
    k = torch.randn((1, 8, 512, 64), generator=g).to(dev)
    v = torch.randn((1, 8, 512, 64), generator=g).to(dev)
    cos, sin = build_rope_cos_sin(precompute_freqs_cis(64, 512), torch.float32, dev)
    flops = 4.0 * 32 * 512 * 512 * 64 / 2

    def step():   # q's RoPE inside the attention kernel, K's by apply_rotary
        return flash_attention(q, apply_rotary(k, cos, sin), v, return_lse=True,
                               rope_cos=cos, rope_sin=sin)
    _settle(torch, step, warmup)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    return {"config": "1: fp32 RoPE (theta 5e5) on Q/K + causal GQA prefill B1 S512 32/8 D64",
            "value": round(flops / (ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": ms, "flops": flops}


def bench_prefill_model_layout(torch, steps: int, warmup: int) -> dict:
    """Config 2's attention block as the model runs it (src/model.py Attention,
    the reference's src/model.py:57-79): q/k/v are views of [B, S, H, D]
    projection outputs, RoPE(K) + V are appended to a KV cache of capacity
    4096, and attention reads q (RoPE'd in the kernel's Q prologue) against the
    cache views.  Also timed: the same with RoPE(q) as its own launch
    (apply_rotary, the reference's sequence)."""
    from src.config import ModelArgs
    from src.flash_attn import flash_attention
    from src.kv_cache import KVCache
    from src.rope import DeviceRopeTable, apply_rotary, precompute_freqs_cis, rope_and_cache_update
    dev = torch.device("cuda:0")
    B, S, Hq, Hkv, D, T = 4, 2048, 32, 8, 64, 4096
    args = ModelArgs(dim=Hq * D, n_layers=1, n_heads=Hq, n_kv_heads=Hkv, max_batch_size=B,
                     max_seq_len=T, device=str(dev))
    kv = KVCache(args, dtype=torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)

    def proj(h):
        return torch.randn((B, S, h * D), device=dev, generator=g).to(torch.bfloat16) \
            .view(B, S, h, D).transpose(1, 2)
    xq, xk, xv = proj(Hq), proj(Hkv), proj(Hkv)
    cos, sin = DeviceRopeTable(precompute_freqs_cis(D, T), torch.bfloat16, dev).rows(0, S)
    flops = 4.0 * B * Hq * S * S * D / 2

    def fused(i):
        ck, cv = rope_and_cache_update(xk, xv, cos, sin, kv, 0, start_pos=0)
        return flash_attention(xq, ck, cv, rope_cos=cos, rope_sin=sin)

    def separate(i):
        q = apply_rotary(xq, cos, sin)
        ck, cv = rope_and_cache_update(xk, xv, cos, sin, kv, 0, start_pos=0)
        return flash_attention(q, ck, cv)

    def append_only(i):
        return rope_and_cache_update(xk, xv, cos, sin, kv, 0, start_pos=0)
    res = {}
    # several calls per graph, so the host's replay submission is not what is timed
    for name, fn, n in (("fused", fused, 4), ("separate_q_rope", separate, 4),
                        ("rope_k_append", append_only, 16)):
        graph = _graph_decode(torch, fn, n)
        res[name] = _time_graph(torch, graph, n, max(steps, 4 * n), warmup)
        del graph
    ms = res["fused"]
    kbytes = B * Hkv * S * D * 2 * 4  # K and V read, RoPE(K) and V written
    return {"config": "2 in the model layout: RoPE(K) + KV append (T 4096) + attention with "
                      "RoPE(q) in the kernel, q/k/v views of [B,S,H,D] projections",
            "value": round(flops / (ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s", "ms_per_step": ms,
            "flops": flops,
            "separate_q_rope": {"ms_per_step": res["separate_q_rope"],
                                "value": round(flops / (res["separate_q_rope"] * 1e-3) / 1e12, 1)},
            "rope_k_append": {"ms": res["rope_k_append"], "bytes": kbytes,
                              "GB/s": round(kbytes / (res["rope_k_append"] * 1e-3) / 1e9, 1)}}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one plain 1 GiB device copy (scales rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--only", choices=["prefill", "prefill_model", "decode", "step", "gemm", "e2e",
                                       "load"],
                    default=None,
                    help="run one leg only (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n}))
        return

    extra = {}
    pre = None
    if args.only in (None, "prefill"):
        pre = bench_prefill(torch, args.steps, args.warmup)
        extra["prefill_config1"] = bench_prefill_cfg1(torch, args.steps, args.warmup)
        extra["prefill_d128"] = bench_prefill_d128(torch, args.steps, args.warmup)
    if args.only in (None, "prefill_model"):
        extra["prefill_config2_model_layout"] = bench_prefill_model_layout(torch, args.steps,
                                                                           args.warmup)
    if args.only in (None, "decode"):
        extra["decode_config3"] = bench_decode_cfg3(torch, args.steps, args.warmup)
        extra["decode_config4"] = bench_decode_cfg4(torch, args.steps, args.warmup)
    if args.only in (None, "step"):
        extra["decode_step_config5"] = bench_config5(torch, args.steps, args.warmup)
    if args.only in (None, "gemm"):
        extra["w8a16_prefill_gemm"] = bench_w8a16_prefill(torch, args.steps, args.warmup)
    if args.only in (None, "e2e"):
        extra["w8a16_prefill_model"] = bench_w8a16_prefill_e2e(torch, args.steps, args.warmup)
    if args.only == "load":    # host I/O; not part of the default run
        extra["checkpoint_load"] = bench_loader(torch)
    cpu = None
    if not args.no_cpu_baseline and args.only is None:
        cpus = cpu_baselines(torch)
        cpu = cpus["config2"]
        for key, leg in (("config1", "prefill_config1"), ("config3", "decode_config3"),
                         ("config4", "decode_config4"), ("config5", "decode_step_config5")):
            if leg in extra:
                extra[leg]["cpu_baseline"] = cpus[key]
    line = {
        "metric": "flash-decode HBM GB/s (% of peak) + prefill attn TFLOP/s, 1 MI355X",
        "value": round(pre["value"], 1) if pre else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms_per_step"], 4) if pre else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) inputs (torch.Generator seed 0), no checkpoint",
        "config": {"workload": "config 2: causal GQA prefill B4 S2048 Hq32 Hkv8 D64, "
                               "bf16 in/out, fp32 accumulate + fp32 LSE",
                   "batch": 4, "seq_len": 2048, "n_heads": 32, "n_kv_heads": 8,
                   "head_dim": 64, "flops_per_step": pre["flops"] if pre else None},
        "roofline": pre["roofline"] if pre else None,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
