"""Standalone kernel measurements on one MI355X.

    python -m nutllm_amd.kernel_bench [--iters N]

* Quantised matvec (nut_matvec_q, matvec_quantized_threaded in the
  reference, src/quant.cpp:257-321) for the five standalone shapes, INT4 and
  INT8, x ~ N(0, 1), W ~ N(0, 0.02) (seed 2). Each timed loop rotates through
  enough distinct uploaded copies of W (at least 300 MB) that the 256 MB
  MALL cannot hold them. Algorithmic bytes = packed weights + fp16 scales +
  4 in (x) + 4 out (y); GB/s = bytes / average launch time from HIP events
  on the launch stream; the roofline is the 8 TB/s HBM peak.
* fp32 GEMM 768 x 768 x 768 (nut_matmul_f32, matmul_threaded,
  src/threading.cpp:163-181), A, B ~ N(0, 1): 905,969,664 FLOP per call
  against the 157.3 TFLOP/s fp32 matrix peak.

Prints one JSON object per measurement.
"""
from __future__ import annotations

import argparse
import json

import numpy as np

from . import (DeviceArray, INT4, INT8, QWeight, Timer, check, device_count,
               lib, quantize, synth_normal, workloads)

HBM_PEAK_GBS = 8000.0
FP32_MATRIX_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 300 << 20


def matvec_case(rows, cols, qtype, index, iters):
    w = synth_normal(workloads.MATVEC_SEED, 100 + index, rows * cols).reshape(
        rows, cols)
    x = synth_normal(workloads.MATVEC_SEED, 200 + index, cols, sigma=1.0)
    data, scales = quantize(w, qtype)
    weight_bytes = data.nbytes + scales.nbytes
    copies = max(2, -(-ROTATE_BYTES // weight_bytes))
    mats = [QWeight(data, scales, rows, cols, qtype) for _ in range(copies)]
    dx = DeviceArray(like=x)
    dy = DeviceArray(4 * rows)
    for m in mats[:4]:
        m.matvec(dx, dy)
    timer = Timer()
    launches = max(iters, copies)
    timer.begin()
    for i in range(launches):
        mats[i % copies].matvec(dx, dy)
    ms = timer.end()
    per_launch_s = ms * 1e-3 / launches
    algorithmic = weight_bytes + 4 * cols + 4 * rows
    gbs = algorithmic / per_launch_s / 1e9
    for m in mats:
        m.close()
    dx.close()
    dy.close()
    return {
        "kernel": "matvec_q", "shape": [rows, cols],
        "type": "int4" if qtype == INT4 else "int8",
        "bytes_per_launch": algorithmic, "copies_rotated": copies,
        "us_per_launch": round(per_launch_s * 1e6, 3),
        "GBps": round(gbs, 1), "roofline_frac": round(gbs / HBM_PEAK_GBS, 4),
    }


def gemm_case(n, iters):
    a = synth_normal(7, 1, n * n, sigma=1.0)
    b = synth_normal(7, 2, n * n, sigma=1.0)
    da, db, dc = DeviceArray(like=a), DeviceArray(like=b), DeviceArray(4 * n * n)
    for _ in range(3):
        check(lib().nut_matmul_f32(da.ptr, db.ptr, dc.ptr, n, n, n, None))
    timer = Timer()
    timer.begin()
    for _ in range(iters):
        check(lib().nut_matmul_f32(da.ptr, db.ptr, dc.ptr, n, n, n, None))
    ms = timer.end()
    flop = 2 * n ** 3
    per_call = ms * 1e-3 / iters
    tflops = flop / per_call / 1e12
    da.close(), db.close(), dc.close()
    return {
        "kernel": "matmul_f32", "shape": [n, n, n], "flop_per_call": flop,
        "us_per_call": round(per_call * 1e6, 2), "TFLOPs": round(tflops, 2),
        "roofline_frac": round(tflops / FP32_MATRIX_PEAK_TFLOPS, 4),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=200)
    args = ap.parse_args()
    if device_count() < 1:
        raise SystemExit("no gfx950 device")
    for i, (rows, cols) in enumerate(workloads.MATVEC_SHAPES):
        for qtype in (INT4, INT8):
            print(json.dumps(matvec_case(rows, cols, qtype, i, args.iters)),
                  flush=True)
    print(json.dumps(gemm_case(768, args.iters)), flush=True)


if __name__ == "__main__":
    main()
