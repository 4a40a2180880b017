"""Headline benchmark: Llama-3-8B-shaped Q4_0 batch-1 decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

One step = one decode step (one token) of the hipGraph-captured HIP decode path: embed,
32 x [RMSNorm+QKV GEMV, RoPE+KV append+split-K attention, o_proj+residual, RMSNorm+gate/up+SwiGLU,
down+residual], RMSNorm+LM head+argmax. Weights are random N(0, 0.02) quantized to Q4_0 on the
device (synthetic; no checkpoint), the prompt is 128 seeded random token ids (prefilled through the
same graph, untimed), then W untimed and K timed greedy decode steps: the default W=5, K=251 covers
the 256 decode steps of benchmark configuration 2 (positions 128..383). Inputs are resident in HBM before
the timed region; the region is synchronized on both sides and timed with HIP events on the
graph's stream (host clock reported beside it).

Printed JSON (one line): value = decode tok/s, plus achieved HBM GB/s from the algorithmic bytes
per step, the roofline of the dominant kernel (fused gate/up GEMV, timed alone with events) and
the CPU oracle timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s + achieved HBM GB/s (% of ~8 TB/s), Llama-3-8B Q4 bs=1, 1 GPU"
HBM_PEAK_GBPS = 8000.0


def _step_ms(rep: dict, steps: int) -> dict:
    """Per-step device time of the timed graph replays (an event after every step): mean, median,
    99th percentile (nearest rank) and maximum, in ms."""
    return {"mean": round(rep["decode_ms"] / max(steps, 1), 5), "p50": round(rep["step_p50_ms"], 5),
            "p99": round(rep["step_p99_ms"], 5), "max": round(rep["step_max_ms"], 5)}
PROMPT_LEN = 128
# HBM bytes per launch of the dominant kernel, measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# and scaled by a copy kernel of known size; the file records the commands and the raw counters.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_gemv_hbm_traffic.md")


def measured_traffic() -> int | None:
    """`traffic_bytes_per_launch = N` from the committed counter summary, if present."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch ="):
                    return int(line.split("=", 1)[1].strip().split()[0])
    except OSError:
        return None
    return None


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _usable_cores() -> int:
    """Cores this process may run on, capped by OMP_NUM_THREADS where the host sets it."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(n, 1)


def cpu_baseline(seed: int, tokens: int = 3) -> dict:
    """The CPU oracle (fp32, Q4_0 rows dequantized on the fly, AVX2/FMA, bf16 KV) running the whole
    32-layer Llama-3-8B-shaped model: one untimed token, then `tokens` timed tokens on one thread
    (the reference engine is single-threaded, src/runtime.rs:702-740) and the same on every usable
    core (the reference's OpenMP C99 module, src/codegen.rs:208-213). tok/s = tokens / seconds."""
    from oracle import pyoracle as po

    cfg = dict(vocab_size=128256, hidden_dim=4096, intermediate_dim=14336, num_layers=32, num_heads=32,
               num_kv_heads=8, head_dim=128, max_seq_len=2 * tokens + 4, rms_norm_eps=1e-5,
               rope_theta=500000.0, qkv_bias=0, tied_lm_head=0)
    cores = _usable_cores()
    t0 = time.perf_counter()
    eng = po.Engine(cfg, seed=seed, q4_0=True, kv_bf16=True, threads=cores)
    gen_s = time.perf_counter() - t0
    prompt = po.prompt_tokens(seed, 2 * tokens + 2, cfg["vocab_size"])

    def tok_per_s(threads: int, pos0: int) -> float:
        eng.set_threads(threads)
        eng.forward(int(prompt[pos0]), pos0)  # untimed: first touch of the activations at this thread count
        t = time.perf_counter()
        for i in range(1, tokens + 1):
            eng.forward(int(prompt[pos0 + i]), pos0 + i)
        return tokens / (time.perf_counter() - t)

    tok_s_1 = tok_per_s(1, 0)
    tok_s_n = tok_per_s(cores, tokens + 1)
    eng.close()
    return {
        "value": round(tok_s_1, 4), "unit": "tok/s", "cores": 1, "kind": "port",
        "sample": (f"CPU oracle (restatement of src/runtime.rs forward_step: fp32, Q4_0 rows dequantized on the fly, "
                   f"AVX2/FMA, bf16 KV) on the full 32-layer Llama-3-8B-shaped model with the same synthetic "
                   f"weights: {tokens} timed decode tokens after one untimed, positions 1-{tokens} (1 thread) and "
                   f"{tokens + 2}-{2 * tokens + 1} (all cores)"),
        "all_cores_value": round(tok_s_n, 4), "all_cores": cores,
        "cpu_model": _cpu_model(), "nproc": os.cpu_count(), "model_build_s": round(gen_s, 2),
    }


# The other BASELINE configurations, timed beside the headline on the same box (hipGraph replays of
# the same runner flow): (key, builtin model, seeded context, batch, warmup, timed steps).
OTHER_CONFIGS = (
    ("config1_smollm_135m_fp32_b1", "smollm_135m", 0, 1, 5, 64),
    ("config1_smollm_135m_group64_b1", "smollm_135m", 0, 1, 5, 64),
    ("config3_qwen2_5_7b_ctx2048_b1", "qwen2_5_7b", 2048, 1, 3, 30),
    ("config3_qwen2_5_7b_ctx2048_b8", "qwen2_5_7b", 2048, 8, 3, 20),
    ("config3_qwen2_5_7b_ctx2048_b32", "qwen2_5_7b", 2048, 32, 3, 20),
    ("config5_qwen2_72b_ctx8192_b1", "qwen2_72b", 8192, 1, 3, 15),
)
MLA_CONFIGS = (("config4_deepseek_v3_mla_ctx4096_b1", 1), ("config4_deepseek_v3_mla_ctx4096_b16", 16))
# configuration 4 runs DeepSeek-V3's own stack of attention layers (NUM_LAYERS of
# examples/deepseek_v3_mla.vlx): every layer's 187 MB of fp8 weights stream from HBM once per step,
# where one replayed layer would leave most of them in the 256 MB memory-side cache between replays
MLA_LAYERS = 61


def other_configs(seed: int) -> dict:
    """Benchmark configurations 1 and 3-5 at their stated shapes: decode tokens/s over all sequences (MLA:
    device microseconds per layer step) and the achieved HBM bytes per second of the whole step
    (weights once per step, every sequence's K/V or latent rows)."""
    from velox_amd.engine import mla_run, run

    out = {}
    for key, model, ctx, batch, warmup, steps in OTHER_CONFIGS:
        t0 = time.perf_counter()
        # configuration 1: the reference's fp32 weights, as fp32 rows or converted to its group-64
        # format (its runner's --quantize q4_0), after a 32-token prompt
        unq = 1 if "fp32" in key else 3 if "group64" in key else 0
        cfg1 = unq != 0
        rep, _ = run(model, prompt_len=32 if cfg1 else 1, warmup=warmup, steps=steps, seed=seed, use_graph=True,
                     kernel_passes=0, context_len=ctx, batch=batch, unquantized=unq)
        out[key] = {"value": round(rep["tok_per_s"], 2), "unit": "tok/s", "batch": batch, "context_tokens": ctx,
                    "timed_positions": ([32 + warmup, 31 + warmup + steps] if cfg1 else
                                        [ctx + 1 + warmup, ctx + warmup + steps]),
                    "hbm_gbps": round(rep["hbm_gbps"], 1), "hbm_frac": round(rep["hbm_gbps"] / HBM_PEAK_GBPS, 4),
                    "bytes_per_step": int(rep["bytes_per_step"]), "ms_per_step": round(rep["decode_ms"] / steps, 5),
                    "step_ms": _step_ms(rep, steps)}
        print(f"[bench] {key}: {rep['tok_per_s']:.1f} tok/s, {rep['hbm_gbps']:.0f} GB/s "
              f"({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    for key, batch in MLA_CONFIGS:
        r = mla_run(batch=batch, context_len=4096, warmup=3, steps=10, seed=seed, layers=MLA_LAYERS)
        out[key] = {"value": round(r["us_per_layer"], 3), "unit": "us/layer", "higher_is_better": False,
                    "batch": batch, "context_tokens": 4096, "hbm_gbps": round(r["hbm_gbps"], 1),
                    "hbm_frac": round(r["hbm_gbps"] / HBM_PEAK_GBPS, 4), "bytes_per_step": int(r["bytes_per_layer"]),
                    "attention_us": round(r["attn_us"], 3), "layers": MLA_LAYERS}
        print(f"[bench] {key}: {r['us_per_layer']:.2f} us/layer", file=sys.stderr, flush=True)
    return out


def bench_mla(args) -> int:
    """Benchmark configuration 4: the DeepSeek-V3 absorbed-MLA layer (fp8 e4m3 weights with 128x128 block
    scales, bf16 latent cache of `context_len` seeded positions per sequence and layer), timed as
    hipGraph replays of the decode step over `--mla-layers` layers; value = device microseconds per
    layer (lower is better)."""
    from velox_amd.engine import mla_run

    ctx = args.context_len or 4096
    print(f"[bench] deepseek_v3_mla layer: batch {args.batch}, context {ctx}, warmup {args.warmup}, "
          f"steps {args.steps}", file=sys.stderr, flush=True)
    if args.no_graph:
        return bench_mla_eager(args, ctx)
    r = mla_run(batch=args.batch, context_len=ctx, warmup=args.warmup, steps=args.steps, seed=args.seed,
                layers=args.mla_layers)
    attn_gbps = r["attn_bytes"] / (r["attn_us"] * 1e3) if r["attn_us"] > 0 else 0.0
    print(f"[bench] mla done: {r['us_per_layer']:.2f} us/layer, {r['hbm_gbps']:.0f} GB/s; attention "
          f"{r['attn_us']:.2f} us", file=sys.stderr, flush=True)
    out = {
        "metric": f"MLA layer us + achieved HBM GB/s, DeepSeek-V3 MLA fp8 bs={args.batch} ctx {ctx}, 1 GPU",
        "value": round(r["us_per_layer"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["us_per_layer"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3 x f16 -> f32 (bf16 latent cache)",
        "data": "synthetic",
        "config": {"workload": f"deepseek_v3_mla_fp8_layer_bs{args.batch}_ctx{ctx}", "batch": args.batch,
                   "context_tokens": ctx, "layers": args.mla_layers, "hipgraph": True},
        "hbm_gbps": round(r["hbm_gbps"], 1),
        "hbm_frac": round(r["hbm_gbps"] / HBM_PEAK_GBPS, 4),
        "bytes_per_step": int(r["bytes_per_layer"]),
        "wall_ms": round(r["wall_ms"], 3),
        "roofline": {
            "kernel": "vx_mla_attn_kernel<512,64,4,2> (absorbed MLA attention over the bf16 latent cache, MFMA)",
            "bound": "hbm",
            "achieved": round(attn_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "avg_us": round(r["attn_us"], 3),
            "bytes_per_launch": int(r["attn_bytes"]),
        },
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_mla_eager(args, ctx: int) -> int:
    """The same step launched eagerly (one synchronized step per call), for per-kernel traces:
    rocprofv3's kernel trace of replayed hipGraphs is not usable here. Its wall time includes host
    launch and synchronization, so it is reported beside, never as, the graph figure."""
    import numpy as np

    from velox_amd.engine import MlaEngine

    n = args.warmup + args.steps
    layers = max(args.mla_layers, 1)
    e = MlaEngine("deepseek_v3_mla", max_seq_len=ctx + n + 1, max_batch=args.batch, seed=args.seed,
                  num_layers=layers)
    for b in range(args.batch):
        for layer in range(layers):
            e.fill_cache(layer, b, ctx, seed=args.seed + b)
        e.set_position(b, ctx)
    e.set_hidden(np.random.default_rng(args.seed).standard_normal((args.batch, e.cfg.hidden_dim)).astype(np.float32))
    step = (lambda: e.decode_step(args.batch)) if layers > 1 else (lambda: e.step(0, args.batch))
    for _ in range(args.warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    wall_us = (time.perf_counter() - t0) * 1e6 / max(args.steps, 1) / layers
    e.close()
    print(f"[bench] mla eager: {args.steps} synchronized steps of {layers} layers, {wall_us:.1f} us wall per layer",
          file=sys.stderr, flush=True)
    print(json.dumps({"metric": f"MLA layer eager wall us, DeepSeek-V3 MLA fp8 bs={args.batch} ctx {ctx}, 1 GPU",
                      "value": round(wall_us, 3), "unit": "us/layer (eager, host-synchronized)", "n_gpus": 1,
                      "steps": args.steps, "warmup": args.warmup, "higher_is_better": False, "data": "synthetic",
                      "config": {"workload": f"deepseek_v3_mla_fp8_layer_bs{args.batch}_ctx{ctx}", "hipgraph": False}}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=251)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--kernel-passes", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip benchmark configurations 1 and 3-5, timed beside the headline as other_configs")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--mla-layers", type=int, default=MLA_LAYERS,
                    help="--model deepseek_v3_mla: layers of the timed decode step (1: one replayed layer)")
    ap.add_argument("--prompt-len", type=int, default=PROMPT_LEN)
    ap.add_argument("--model", default="llama3_8b",
                    choices=["llama3_8b", "qwen2_5_7b", "qwen2_72b", "smollm_135m", "deepseek_v3_mla"],
                    help="builtin configuration (the headline metric is llama3_8b; deepseek_v3_mla times one "
                         "absorbed-MLA layer with fp8 weights, benchmark configuration 4)")
    ap.add_argument("--context-len", type=int, default=0,
                    help="start from a seeded context of N positions already in the KV cache (prompt = 1 token)")
    ap.add_argument("--batch", type=int, default=1,
                    help="decode B <= 32 independent sequences per step (batched MFMA GEMMs); value = all tokens/s")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="afterwards run a device-to-device copy of MIB MiB (byte-counter yardstick)")
    ap.add_argument("--prefill-chunk", type=int, default=128,
                    help="beside the headline, time the prompt's batched prefill in chunks of N positions "
                         "(velox_hip_prefill_batch; 0 skips it)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures the single-GPU decode step only; --gpus {args.gpus} is not supported "
              "(this build runs on one GPU: no collectives, no sharding)", file=sys.stderr)
        return 2

    from velox_amd import _lib as L
    from velox_amd.engine import run

    L.load()
    if args.model == "deepseek_v3_mla":
        return bench_mla(args)
    plen = 1 if args.context_len else args.prompt_len
    ctx = args.context_len
    cfg = L.builtin_config(args.model)
    print(f"[bench] {args.model} Q4_0 decode: context {ctx}, prompt {plen}, warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    rep, toks = run(args.model, prompt_len=plen, warmup=args.warmup, steps=args.steps, seed=args.seed,
                    use_graph=not args.no_graph, kernel_passes=args.kernel_passes, context_len=ctx,
                    batch=args.batch)
    print(f"[bench] decode done: {rep['tok_per_s']:.1f} tok/s, {rep['hbm_gbps']:.0f} GB/s; gate/up kernel "
          f"{rep['kernel_us']:.2f} us", file=sys.stderr, flush=True)

    headline = args.model == "llama3_8b" and ctx == 0 and args.batch == 1
    prefill = None
    if headline and args.prefill_chunk > 1:
        # time to first token with the batched prefill, same prompt, against the token-by-token
        # prefill of the run above (the reference runner's flow)
        rep_p, toks_p = run(args.model, prompt_len=plen, warmup=0, steps=1, seed=args.seed,
                            use_graph=not args.no_graph, prefill_chunk=args.prefill_chunk)
        prefill = {"prompt_tokens": plen, "chunk": args.prefill_chunk,
                   "token_by_token_ms": round(rep["prefill_ms"], 3), "batched_ms": round(rep_p["prefill_ms"], 3),
                   "first_token_equal": toks_p[plen - 1] == toks[plen - 1]}
        print(f"[bench] batched prefill: {rep_p['prefill_ms']:.2f} ms vs {rep['prefill_ms']:.2f} ms token by token",
              file=sys.stderr, flush=True)

    if args.copy_calibration > 0:
        L.device_copy_calibration(args.copy_calibration << 20)
    kernel_gbps = rep["kernel_bytes"] / (rep["kernel_us"] * 1e-6) / 1e9 if rep["kernel_us"] > 0 else 0.0
    workload = f"{args.model}_q4_0_decode_bs{args.batch}" + (f"_ctx{ctx}" if ctx else "")
    out = {
        "metric": METRIC if headline else f"decode tok/s + achieved HBM GB/s, {args.model} Q4_0 bs={args.batch}"
                  + (f" ctx {ctx}" if ctx else "") + ", 1 GPU",
        "value": round(rep["tok_per_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(rep["decode_ms"] / max(args.steps, 1), 5),
        "step_ms": _step_ms(rep, args.steps),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("q4_0 x 22-bit block-scaled integer activations -> exact int32 block dots, f32 sums (bf16 KV)"
                  if args.batch == 1 else "q4_0 x f16 -> f32 (bf16 KV)"),
        "data": "synthetic",
        "config": {
            "workload": workload,
            "batch": args.batch,
            "context_tokens": ctx,
            "prompt_tokens": plen,
            "timed_positions": [ctx + plen + args.warmup, ctx + plen + args.warmup + args.steps - 1],
            "hipgraph": not args.no_graph,
        },
        "hbm_gbps": round(rep["hbm_gbps"], 1),
        "hbm_frac": round(rep["hbm_gbps"] / HBM_PEAK_GBPS, 4),
        "bytes_per_step": int(rep["bytes_per_step"]),
        "wall_ms": round(rep["wall_ms"], 3),
        "prefill_ms": round(rep["prefill_ms"], 3),
        "roofline": {
            "kernel": (f"vx_gemv_q4_kernel<S,SWIGLU> (RMSNorm + gate/up Q4_0 GEMV + SwiGLU), "
                       f"{cfg.intermediate_dim}x2 x {cfg.hidden_dim}") if args.batch == 1 else
                      (f"vx_mgemm_kernel<SWIGLU,MT,NT> (gate/up Q4_0 MFMA GEMM + SwiGLU, {args.batch} sequences), "
                       f"{cfg.intermediate_dim}x2 x {cfg.hidden_dim}"),
            "bound": "hbm",
            "achieved": round(kernel_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(kernel_gbps / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic() if headline else None,
            "avg_us": round(rep["kernel_us"], 3),
            "bytes_per_launch": int(rep["kernel_bytes"]),
        },
        "first_tokens": toks[plen - 1:plen + 7],  # ring entries from position ctx on
    }
    if prefill:
        out["prefill"] = prefill
    if not args.no_other_configs and headline:
        out["other_configs"] = other_configs(args.seed)
    if not args.no_cpu_baseline and headline:
        print("[bench] cpu baseline (oracle, bounded sample)...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(args.seed)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
