"""Standalone kernel measurements on one MI355X.

    python -m nutllm_amd.kernel_bench [--iters N]

Runs nutllm_amd/lib/nut_kernel_bench (built from
nutllm_amd/bench/kernel_bench.cpp by the package Makefile), which times the
quantised matvec (5 shapes x INT4/INT8, weights rotated past the MALL) and
the 768^3 fp32 GEMM through the C ABI with launches issued back to back
from C++, and prints one JSON object per measurement.
"""
from __future__ import annotations

import os
import subprocess
import sys

BINARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                      "nut_kernel_bench")


def main():
    if not os.path.exists(BINARY):
        raise SystemExit(f"{BINARY} is not built; run __graft_entry__.build()")
    return subprocess.call([BINARY] + sys.argv[1:])


if __name__ == "__main__":
    sys.exit(main())
