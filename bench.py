#!/usr/bin/env python3
"""bench.py — decode throughput of the gfx950 token loop on one MI355X.

Workload (a "step"): one greedy generate_tokens_cached call
(src/generate.cpp:174-216) on the TinyLlama-1.1B-shaped decoder with random
N(0, 0.02) weights (seed 3), INT4 block-32 linears, fp32 embeddings and
classifier: a 5-token prompt, then 16 greedy tokens. Weights and KV cache are
resident in HBM before the timed region.

value     decode tok/s with the reference's GenerationStats semantics
          (every classifier + argmax + decode step after the prefill).
roofline  algorithmic bytes of the decode loop (packed weights + fp16 scales
          + fp32 classifier + norms + one embedding row per token, plus K/V
          reads) / device time of the decode loop from HIP events on the
          model's stream, against the 8 TB/s HBM peak.
cpu_baseline  the compiled reference's own threaded generate_tokens_cached
          (oracle/_ref, "reference") or, when that library is absent, this
          repo's C restatement ("port"), timed on this host in the same run.

One JSON line goes to stdout; progress to stderr.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PUBLISHED_DECODE_TOK_S = 17.089  # reference, TinyLlama INT4, 4 threads

# HBM bytes one generate launch (16 iterations) moves, from rocprofv3
# counter runs of this bench: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 KiB (the
# scales read off a 1 GiB device-to-device copy in the same runs).
MEASURED_TRAFFIC_BYTES = 13_535_426_731
CPU_SAMPLE_SECONDS = 10.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_bytes_per_position(cfg):
    kv = cfg.kv_heads or cfg.heads
    return 2 * cfg.layers * kv * cfg.head_dim * 4


def cpu_baseline(model, prompt, gen):
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    if oracle.ref_available():
        kind = "reference"
        rm = oracle.RefModel.from_quantized(model)
        run = lambda: rm.generate(prompt, gen, threads)  # noqa: E731
    else:
        kind = "port"
        oracle.orc().orc_set_threads(threads)
        om = oracle.oracle_model(model)
        run = lambda: om.generate(prompt, gen)  # noqa: E731
    rates, prefill = [], []
    ids = None
    start = time.perf_counter()
    # repeat whole generate calls for about CPU_SAMPLE_SECONDS (at most 30)
    while len(rates) < 30 and (len(rates) < 2 or time.perf_counter() - start
                               < CPU_SAMPLE_SECONDS):
        ids, pre, dec = run()
        rates.append(len(ids) / dec)
        prefill.append(len(prompt) / pre)
    elapsed = time.perf_counter() - start
    return {
        "value": round(statistics.median(rates), 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": kind,
        "sample": (f"TinyLlama-shape INT4 greedy generate, {len(prompt)}-token "
                   f"prompt + {gen} tokens, median of {len(rates)} runs "
                   f"({elapsed:.1f} s), {threads} threads; prefill "
                   f"{statistics.median(prefill):.3f} tok/s"),
    }, ids


def long_prompt(args, nut, workloads):
    """Prefill (batched GEMM path) and decode tok/s of a long-prompt run."""
    t = time.time()
    model, prompt, gen = workloads.build_run(args.workload)
    log(f"built synthetic model in {time.time() - t:.1f}s")
    dev = model.to_device()
    cfg = model.config
    if args.path == "steps":
        dev.set_path(nut.PATH_STEPS)
    if args.prefill_only:
        # the batched prefill alone (no decode loop, no captured graph), for
        # kernel traces of the prefill kernels
        cache = nut.KVCache(cfg)
        times = []
        for i in range(args.warmup + args.steps):
            t0 = time.time()
            dev.prefill(cache, prompt)
            if i >= args.warmup:
                times.append(time.time() - t0)
        cache.close()
        dev.close()
        prefill_s = statistics.median(times)
        print(json.dumps({
            "workload": args.workload, "prompt_tokens": len(prompt),
            "steps": args.steps, "warmup": args.warmup, "prefill_only": True,
            "prefill_tok_s": round(len(prompt) / prefill_s, 1),
            "prefill_ms": round(prefill_s * 1e3, 2), "dtype": "fp32",
            "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        }), flush=True)
        return
    for _ in range(args.warmup):
        dev.generate(prompt, gen)
    pre, dec, toks, dms = [], [], 0, []
    for _ in range(args.steps):
        ids, st = dev.generate(prompt, gen)
        pre.append(st.prefill_seconds)
        dec.append(st.decode_seconds)
        dms.append(dev.last_decode_ms())
        toks += st.generated_tokens
    dev.close()
    n = len(ids)
    # the greedy ids the reference generated for this run (tests/golden)
    golden = os.path.join(ROOT, "tests", "golden", f"{args.workload}.npz")
    ref_ids = None
    if os.path.exists(golden):
        import numpy as np
        ref_ids = np.load(golden)["ids"].tolist()
    prefill_s = statistics.median(pre)
    linear = sum(2 * r * c for r, c in nut.projection_shapes(cfg).values())
    kv = cfg.kv_heads or cfg.heads
    attn = sum(4 * cfg.heads * cfg.head_dim * (i + 1) for i in range(len(prompt)))
    flop = len(prompt) * linear * cfg.layers + attn * cfg.layers
    print(json.dumps({
        "workload": args.workload, "prompt_tokens": len(prompt),
        "generated_tokens": n, "steps": args.steps, "warmup": args.warmup,
        "prefill_tok_s": round(len(prompt) / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 2),
        "prefill_tflops": round(flop / prefill_s / 1e12, 2),
        "decode_tok_s": round(toks / sum(dec), 2),
        "decode_device_us_per_token": round(statistics.median(dms) * 1e3 / n, 1),
        "kv_heads": kv, "dtype": "fp32",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "ids_match_reference": None if ref_ids is None else ids == ref_ids,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--workload", default="tinyllama_int4",
                    choices=["tinyllama_int4", "tinyllama_int8_2k",
                             "llama7b_int4"],
                    help="tinyllama_int4 (default): the headline line below; "
                         "the others print one line of prefill and decode "
                         "tok/s for the long-prompt configurations")
    ap.add_argument("--prefill-only", action="store_true",
                    help="long-prompt workloads: time the batched prefill "
                         "alone (host clock), for kernel traces")
    ap.add_argument("--path", default="auto", choices=["auto", "steps"],
                    help="steps: eager per-token step kernels only (no token "
                         "kernel, batched prefill or graph replay), for "
                         "profiling the step kernels")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the timed region, copy this many MiB device "
                         "to device (the known-size kernel that scales "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: nutllm_amd has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import nutllm_amd as nut
    from nutllm_amd import workloads

    if nut.device_count() < 1:
        print("no gfx950 device", file=sys.stderr)
        sys.exit(1)
    if args.workload != "tinyllama_int4":
        long_prompt(args, nut, workloads)
        return
    t = time.time()
    model, prompt, gen = workloads.build_run("tinyllama_int4")
    log(f"built synthetic model in {time.time() - t:.1f}s")
    dev = model.to_device()
    cfg = model.config

    for _ in range(args.warmup):
        dev.generate(prompt, gen)
    decode_s, prefill_s, device_ms, tokens = [], [], [], 0
    ids = None
    nut.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ids, st = dev.generate(prompt, gen)
        decode_s.append(st.decode_seconds)
        prefill_s.append(st.prefill_seconds)
        device_ms.append(dev.last_decode_ms())
        tokens += st.generated_tokens
    nut.synchronize()
    t1 = time.perf_counter()
    dev.close()

    value = tokens / sum(decode_s)
    n = len(ids)
    per_pos = kv_bytes_per_position(cfg)
    # each decode-loop iteration at cache length P+i reads K/V of P+i+1
    kv_bytes = sum(per_pos * (len(prompt) + i + 1) for i in range(n))
    step_bytes = model.weight_bytes_per_token() * n + kv_bytes
    achieved = step_bytes / (statistics.median(device_ms) * 1e-3) / 1e9
    line = {
        "metric": "decode tok/s, TinyLlama-1.1B-shape INT4 (greedy, 5-token "
                  "prompt, 16 tokens)",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((t1 - t0) * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / PUBLISHED_DECODE_TOK_S, 3),
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {
            "workload": "TinyLlama-1.1B-shape INT4 block-32 greedy decode",
            "dim": cfg.dim, "layers": cfg.layers, "heads": cfg.heads,
            "kv_heads": cfg.kv_heads, "ffn_dim": cfg.ffn_dim,
            "vocab": cfg.vocab_size, "prompt_tokens": len(prompt),
            "generated_tokens": n,
        },
        "prefill_tok_s": round(len(prompt) / statistics.median(prefill_s), 3),
        "decode_device_us_per_token": round(
            statistics.median(device_ms) * 1e3 / n, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC_BYTES,
            "kernel": "decode loop (classifier + argmax + decode step per "
                      "token)",
            "bytes_per_launch": step_bytes,
        },
    }
    if args.calibrate_copy_mib > 0:
        nbytes = args.calibrate_copy_mib << 20
        src, dst = nut.DeviceArray(nbytes), nut.DeviceArray(nbytes)
        for _ in range(2):
            nut.check(nut.lib().nut_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        src.close(), dst.close()
        log(f"copied {args.calibrate_copy_mib} MiB device to device, twice")
    if not args.no_cpu:
        log("timing the CPU baseline")
        base, cpu_ids = cpu_baseline(model, prompt, gen)
        line["cpu_baseline"] = base
        line["cpu_ids_match"] = cpu_ids == ids
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
