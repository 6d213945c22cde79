#!/usr/bin/env python3
"""bench.py — throughput of the gfx950 token loop on one MI355X.

Default workload (a "step"): one greedy generate_tokens_cached call
(src/generate.cpp:174-216) on the TinyLlama-1.1B-shaped decoder with random
N(0, 0.02) weights (seed 3), INT4 block-32 linears, fp32 embeddings and
classifier: a 5-token prompt, then 16 greedy tokens. Weights and KV cache are
resident in HBM before the timed region.

value     decode tok/s with the reference's GenerationStats semantics
          (every classifier + argmax + decode step after the prefill).
roofline  algorithmic bytes of the decode loop (the model's weight bytes per
          token: packed weights + fp16 scales of every projection, the fp32
          classifier as stored, norms, one embedding row; plus K/V reads) /
          device time of the decode loop from HIP events on the model's
          stream, against the 8 TB/s HBM peak.
          roofline.traffic: HBM bytes per generate launch measured in the same
          run, before the timed region, by two rocprofv3 counter passes
          (FETCH_SIZE, WRITE_SIZE) over a child run of this script, each
          scaled by the counter's reading for a 1 GiB device-to-device copy
          (--no-traffic skips them; traffic is then null); each pass's exit
          status is kept in traffic_counters.
screened_roofline  the same over the bytes the decode loop actually reads:
          the greedy argmax goes through the classifier's INT8 block-32
          screening copy and recomputes fp32 logits only for the few rows
          its error bounds cannot rule out (those rows not counted).
cpu_baseline  the compiled reference's own threaded generate_tokens_cached
          (oracle/_ref, "reference") or, when that library is absent, this
          repo's C restatement ("port"), timed on this host in the same run
          at 1, 4 and the host's physical cores (at most 16, the box's CPU
          share); value is the physical-core figure.

Other workloads (--workload), one JSON line each:
  tinyllama_int8_2k, llama7b_int4
          2048- / 512-token prompt (batched MFMA prefill) then 128 greedy
          tokens: decode tok/s with its HBM roofline (weights + K/V at each
          step's context), prefill tok/s with its MFMA roofline, the
          reference CPU decode loop timed on a bounded sample at the same
          context, and whether the ids equal the reference's
          (tests/golden/<workload>.npz).
  kernels the standalone quantised matvec (5 shapes x INT4/INT8, weights
          rotated past the 256 MB memory-side cache) and the 768^3 fp32
          GEMM, from nutllm_amd/lib/nut_kernel_bench (launches issued from
          C++), each with the reference's matvec_quantized_threaded /
          matmul_threaded timed beside it; one line per kernel and shape.

Progress goes to stderr.
"""
import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0  # dense f16, MI355X
PUBLISHED_DECODE_TOK_S = 17.089  # reference, TinyLlama INT4, 4 threads

CPU_SAMPLE_SECONDS = 8.0
TRAFFIC_PASS_TIMEOUT = 180  # seconds per rocprofv3 counter pass
CALIBRATE_MIB = 1024
MAX_THREADS = 16  # host threads for the CPU baseline (the CPU share of one GPU's host)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_info():
    """CPU model name and physical core count of this host."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                key, value = key.strip(), value.strip()
                if key == "model name":
                    model = value
                elif key == "physical id":
                    phys = value
                elif key == "core id":
                    core = value
                elif not key and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:
        pass
    if phys is not None and core is not None:
        cores.add((phys, core))
    n = len(cores) or (os.cpu_count() or 1)
    return model, n


def counter_pass(counter, workload):
    """One rocprofv3 counter pass over a single generate of `workload` (a
    child process: python3 bench.py under rocprofv3 --pmc COUNTER), plus a
    CALIBRATE_MIB device-to-device copy in the same process. Returns
    (KiB per decode-kernel dispatch, KiB per copy dispatch, the child's exit
    status: negative for a signal)."""
    import glob
    import shutil
    import signal
    import tempfile
    tool = shutil.which("rocprofv3")
    if tool is None:
        raise RuntimeError("rocprofv3 not found")
    out = tempfile.mkdtemp(prefix="nut_pmc_")
    cmd = [tool, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "run", "--",
           sys.executable, os.path.abspath(__file__), "--no-cpu", "--no-traffic",
           "--workload", workload, "--steps", "1", "--warmup", "0",
           "--calibrate-copy-mib", str(CALIBRATE_MIB)]
    proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                            start_new_session=True)
    try:
        proc.wait(timeout=TRAFFIC_PASS_TIMEOUT)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.wait()
        raise RuntimeError(f"{counter} pass timed out")
    # The tool can end with SIGSEGV in exit() after writing complete files;
    # the status is returned with the counts so the line records it.
    files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
    try:
        kernel, copy = parse_counter_csv(files, counter)
        return kernel, copy, proc.returncode
    except RuntimeError as e:
        raise RuntimeError(f"{e} (exit status {proc.returncode})") from None
    finally:
        shutil.rmtree(out, ignore_errors=True)


def parse_counter_csv(files, counter):
    """(mean value per decode-kernel dispatch, value of the largest copy
    dispatch) of `counter` in rocprofv3 counter-collection CSV files. The
    decode kernels are the cooperative generate launches (token_kernel, and
    wide_kernel at the 7B widths); a dispatch's rows (one per counter in the
    files seen here) are summed."""
    import csv
    kernel, copy = {}, {}
    for name in files:
        with open(name, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                key = (name, row.get("Dispatch_Id", ""))
                v = float(row["Counter_Value"])
                k = row.get("Kernel_Name", "")
                if "token_kernel" in k or "wide_kernel" in k:
                    kernel[key] = kernel.get(key, 0.0) + v
                elif "copyBuffer" in k:
                    copy[key] = copy.get(key, 0.0) + v
    if not kernel or not copy:
        raise RuntimeError(f"{counter} pass: no decode-kernel or copy dispatch")
    # the calibration copies are the largest copy dispatches (model upload
    # copies are small)
    return statistics.mean(kernel.values()), max(copy.values())


def measured_traffic(workload):
    """HBM bytes of one generate launch of `workload` from FETCH_SIZE and
    WRITE_SIZE counter passes of this build, each scaled by what the counter
    reads for the CALIBRATE_MIB copy: FETCH_SIZE counts half of a copy's read
    bytes on this GPU, WRITE_SIZE all of its written bytes."""
    true_kib = CALIBRATE_MIB * 1024
    fetch, fetch_copy, fetch_rc = counter_pass("FETCH_SIZE", workload)
    log(f"FETCH_SIZE pass done (exit status {fetch_rc})")
    write, write_copy, write_rc = counter_pass("WRITE_SIZE", workload)
    log(f"WRITE_SIZE pass done (exit status {write_rc})")
    f_scale, w_scale = true_kib / fetch_copy, true_kib / write_copy
    return {"bytes": int(round((fetch * f_scale + write * w_scale) * 1024)),
            "fetch_kib": round(fetch, 1), "fetch_scale": round(f_scale, 5),
            "write_kib": round(write, 1), "write_scale": round(w_scale, 5),
            "fetch_exit_status": fetch_rc, "write_exit_status": write_rc}


def kv_bytes_per_position(cfg):
    kv = cfg.kv_heads or cfg.heads
    return 2 * cfg.layers * kv * cfg.head_dim * 4


def thread_counts():
    model, physical = cpu_info()
    top = max(1, min(physical, MAX_THREADS, os.cpu_count() or 1))
    return model, physical, sorted({1, min(4, top), top})


def cpu_baseline(model, prompt, gen):
    """The reference's generate_tokens_cached at 1, 4 and all physical
    cores (each for about CPU_SAMPLE_SECONDS)."""
    import oracle
    cpu_model, physical, counts = thread_counts()
    if oracle.ref_available():
        kind = "reference"
        rm = oracle.RefModel.from_quantized(model)
        run = lambda t: rm.generate(prompt, gen, t)  # noqa: E731
    else:
        kind = "port"
        om = oracle.oracle_model(model)

        def run(t):
            oracle.orc().orc_set_threads(t)
            return om.generate(prompt, gen)
    by_threads, prefill, ids, total = {}, {}, None, 0.0
    for t in counts:
        rates, pre = [], []
        start = time.perf_counter()
        while len(rates) < 30 and (len(rates) < 2 or time.perf_counter() - start
                                   < CPU_SAMPLE_SECONDS):
            ids, p, d = run(t)
            rates.append(len(ids) / d)
            pre.append(len(prompt) / p)
        total += time.perf_counter() - start
        by_threads[str(t)] = round(statistics.median(rates), 3)
        prefill[str(t)] = round(statistics.median(pre), 3)
    top = str(counts[-1])
    return {
        "value": by_threads[top],
        "unit": "tok/s",
        "cores": counts[-1],
        "kind": kind,
        "cpu_model": cpu_model,
        "physical_cores": physical,
        "by_threads": by_threads,
        "prefill_tok_s_by_threads": prefill,
        "sample": (f"TinyLlama-shape INT4 greedy generate_tokens_cached, "
                   f"{len(prompt)}-token prompt + {gen} tokens, median of up to 30 "
                   f"runs per thread count ({total:.1f} s in all), GenerationStats "
                   f"semantics; value at {top} threads"),
    }, ids


def calibration_copy(args, nut):
    """The known-size copy that scales a counter pass's FETCH_SIZE and
    WRITE_SIZE (--calibrate-copy-mib; nothing when 0)."""
    if args.calibrate_copy_mib > 0:
        nbytes = args.calibrate_copy_mib << 20
        src, dst = nut.DeviceArray(nbytes), nut.DeviceArray(nbytes)
        for _ in range(2):
            nut.check(nut.lib().nut_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        src.close(), dst.close()
        log(f"copied {args.calibrate_copy_mib} MiB device to device, twice")


def add_traffic(line, traffic, traffic_error):
    """roofline.traffic (HBM bytes per generate launch, measured), its ratio
    to the algorithmic bytes and to the bytes the loop reads (screened
    classifier), or the reason it was not measured."""
    roof = line["roofline"]
    if traffic is not None:
        roof["traffic"] = traffic["bytes"]
        roof["traffic_ratio"] = round(traffic["bytes"] / roof["bytes_per_launch"], 4)
        roof["traffic_ratio_bytes_read"] = round(
            traffic["bytes"] / line["screened_roofline"]["bytes_per_launch"], 4)
        roof["traffic_counters"] = traffic
    elif traffic_error is not None:
        roof["traffic_error"] = traffic_error


def decode_rooflines(model_bytes, read_bytes, device_ms, kernel):
    """roofline (the model's weight bytes + K/V per launch over the decode
    loop's device time) and screened_roofline (the bytes the loop reads)."""
    achieved = model_bytes / (device_ms * 1e-3) / 1e9
    read = read_bytes / (device_ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": kernel, "bytes_per_launch": model_bytes,
            "device_ms_per_launch": round(device_ms, 4)}
    screened = {"achieved": round(read, 1), "unit": "GB/s",
                "frac": round(read / HBM_PEAK_GBS, 4), "bytes_per_launch": read_bytes}
    return roof, screened


def long_prompt(args, nut, workloads, traffic=None, traffic_error=None):
    """Prefill (batched GEMM path) and decode of a long-prompt run."""
    import numpy as np
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
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ids, st = dev.generate(prompt, gen)
        pre.append(st.prefill_seconds)
        dec.append(st.decode_seconds)
        dms.append(dev.last_decode_ms())
        toks += st.generated_tokens
    t1 = time.perf_counter()
    dev.close()
    n = len(ids)
    # the greedy ids the reference generated for this run (tests/golden)
    golden = os.path.join(ROOT, "tests", "golden", f"{args.workload}.npz")
    ref_ids = np.load(golden)["ids"].tolist() if os.path.exists(golden) else None
    prefill_s = statistics.median(pre)
    linear = sum(2 * r * c for r, c in nut.projection_shapes(cfg).values())
    attn = sum(4 * cfg.heads * cfg.head_dim * (i + 1) for i in range(len(prompt)))
    flop = len(prompt) * linear * cfg.layers + attn * cfg.layers
    device_ms = statistics.median(dms)
    per_pos = kv_bytes_per_position(cfg)
    kv_bytes = sum(per_pos * (len(prompt) + i + 1) for i in range(n))
    screened = args.path != "steps"  # the token kernels screen the classifier
    read_bytes = model.weight_bytes_per_token(screened=screened) * n + kv_bytes
    model_bytes = model.weight_bytes_per_token() * n + kv_bytes
    roof, screened_roof = decode_rooflines(
        model_bytes, read_bytes, device_ms,
        "decode loop (classifier + argmax + decode step per token)")
    line = {
        "metric": f"decode tok/s, {args.workload} (greedy, {len(prompt)}-token prompt, "
                  f"{gen} tokens)",
        "value": round(toks / sum(dec), 2),
        "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round((t1 - t0) * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8" if model.qtype == 0 else "int4",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {"workload": args.workload, "dim": cfg.dim, "layers": cfg.layers,
                   "heads": cfg.heads, "kv_heads": cfg.kv_heads or cfg.heads,
                   "ffn_dim": cfg.ffn_dim, "vocab": cfg.vocab_size,
                   "prompt_tokens": len(prompt), "generated_tokens": n},
        "decode_device_us_per_token": round(device_ms * 1e3 / n, 1),
        "roofline": roof,
        "screened_roofline": screened_roof,
        "prefill_tok_s": round(len(prompt) / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 2),
        "prefill_roofline": {"bound": "mfma", "achieved": round(flop / prefill_s / 1e12, 1),
                             "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(flop / prefill_s / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
                             "flop": flop},
        "ids_match_reference": None if ref_ids is None else ids == ref_ids,
    }
    add_traffic(line, traffic, traffic_error)
    calibration_copy(args, nut)
    if not args.no_cpu:
        line["cpu_baseline"] = long_cpu_baseline(model, prompt, ids)
    print(json.dumps(line), flush=True)


def long_cpu_baseline(model, prompt, ids):
    """The reference's decode loop (norm, classifier, argmax,
    decode_quantized_token) from the workload's context, on a bounded
    sample; and the same from the prompt's mean position (the reference
    prefills token by token, so that is its prefill rate there)."""
    import oracle
    if not oracle.ref_available():
        return None
    cpu_model, physical, counts = thread_counts()
    threads = counts[-1]
    rm = oracle.RefModel.from_quantized(model)
    toks = list(ids) + [int(t) for t in prompt]
    room = model.config.max_seq - len(prompt)  # the cache holds max_seq rows
    one = rm.decode_time(len(prompt), toks[:1], threads)
    k = max(1, min(len(toks), room, int(15.0 / max(one, 1e-3))))
    dec_s = rm.decode_time(len(prompt), toks[:k], threads)
    mid = len(prompt) // 2
    kp = max(1, min(len(toks), k, model.config.max_seq - mid))
    pre_s = rm.decode_time(mid, toks[:kp], threads)
    rm.close()
    return {
        "value": round(k / dec_s, 3), "unit": "tok/s", "cores": threads,
        "kind": "reference", "cpu_model": cpu_model, "physical_cores": physical,
        "prefill_tok_s": round(kp / pre_s, 3),
        "sample": (f"{k} decode-loop steps of the reference (final rmsnorm, fp32 "
                   f"classifier, argmax, decode_quantized_token) from context "
                   f"{len(prompt)} ({dec_s:.1f} s); prefill rate: {kp} steps from "
                   f"position {mid}, the prompt's mean position ({pre_s:.1f} s); "
                   f"{threads} threads"),
    }


def kernels(args):
    """Standalone kernels (nut_kernel_bench) with the reference beside them."""
    import numpy as np

    import nutllm_amd as nut
    binary = os.path.join(ROOT, "nutllm_amd", "lib", "nut_kernel_bench")
    out = subprocess.run([binary, "--iters", str(max(20, args.steps * 40))],
                         capture_output=True, text=True, check=True).stdout
    lines = [json.loads(x) for x in out.splitlines() if x.startswith("{")]
    ref = None
    if not args.no_cpu:
        import oracle
        ref = oracle.ref() if oracle.ref_available() else None
    cpu_model, physical, counts = thread_counts()
    threads = counts[-1]
    shapes = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (4096, 4096)]
    for m in lines:
        base = None
        if ref is not None and m["kernel"] == "matvec_q":
            rows, cols = m["shape"]
            i = shapes.index((rows, cols))
            w = nut.synth_normal(2, 100 + i, rows * cols, 0.02)
            x = nut.synth_normal(2, 200 + i, cols, 1.0)
            qt = 1 if m["type"] == "int4" else 0
            sec = oracle.C.c_double()
            oracle.check(ref.ref_matvec_q_time(oracle.ptr(w), rows, cols, qt, oracle.ptr(x),
                                               threads, 50, oracle.C.byref(sec)))
            base = {"value": round(m["bytes_per_launch"] / sec.value / 1e9, 2),
                    "unit": "GB/s", "cores": threads, "kind": "reference",
                    "cpu_model": cpu_model,
                    "sample": f"median of 50 matvec_quantized_threaded calls, "
                              f"{threads} threads"}
        elif ref is not None and m["kernel"] == "matmul_f32":
            n = m["shape"][0]
            a = nut.synth_normal(7, 1, n * n, 1.0)
            b = nut.synth_normal(7, 2, n * n, 1.0)
            sec = oracle.C.c_double()
            oracle.check(ref.ref_matmul_time(oracle.ptr(a), oracle.ptr(b), n, n, n,
                                             threads, 5, oracle.C.byref(sec)))
            base = {"value": round(m["flop_per_call"] / sec.value / 1e12, 4),
                    "unit": "TFLOP/s", "cores": threads, "kind": "reference",
                    "cpu_model": cpu_model,
                    "sample": f"median of 5 matmul_threaded calls, {threads} threads"}
        m["cpu_baseline"] = base
        print(json.dumps(m), flush=True)
    del np


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--workload", default="tinyllama_int4",
                    choices=["tinyllama_int4", "tinyllama_int8_2k", "llama7b_int4",
                             "kernels"],
                    help="tinyllama_int4 (default): the headline line; the others "
                         "print the long-prompt lines or the standalone kernels")
    ap.add_argument("--prefill-only", action="store_true",
                    help="long-prompt workloads: time the batched prefill "
                         "alone (host clock), for kernel traces")
    ap.add_argument("--path", default="auto", choices=["auto", "steps"],
                    help="steps: eager per-token step kernels only (no token "
                         "kernel, batched prefill or graph replay), for "
                         "profiling the step kernels")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure "
                         "roofline.traffic")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the timed region, copy this many MiB device "
                         "to device (the known-size kernel that scales "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: nutllm_amd has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    # The counter passes run as child processes before this process touches
    # the GPU (decode workloads on the cooperative generate kernels).
    traffic, traffic_error = None, None
    if (args.workload != "kernels" and not args.prefill_only and args.path != "steps"
            and not args.no_traffic):
        log("measuring HBM traffic (two rocprofv3 counter passes)")
        try:
            traffic = measured_traffic(args.workload)
        except (RuntimeError, OSError, ValueError, KeyError) as e:
            traffic_error = str(e)
            log(f"traffic not measured: {e}")

    import nutllm_amd as nut
    from nutllm_amd import workloads

    if nut.device_count() < 1:
        print("no gfx950 device", file=sys.stderr)
        sys.exit(1)
    if args.workload == "kernels":
        kernels(args)
        return
    if args.workload != "tinyllama_int4":
        long_prompt(args, nut, workloads, traffic, traffic_error)
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
    read_bytes = model.weight_bytes_per_token(screened=True) * n + kv_bytes
    model_bytes = model.weight_bytes_per_token() * n + kv_bytes
    roof, screened_roof = decode_rooflines(
        model_bytes, read_bytes, statistics.median(device_ms),
        "decode loop (classifier + argmax + decode step per token)")
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
        "dtype": "int4",
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
        "roofline": roof,
        "screened_roofline": screened_roof,
    }
    add_traffic(line, traffic, traffic_error)
    calibration_copy(args, nut)
    if not args.no_cpu:
        log("timing the CPU baseline")
        base, cpu_ids = cpu_baseline(model, prompt, gen)
        line["cpu_baseline"] = base
        line["cpu_ids_match"] = cpu_ids == ids
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
