"""Benchmark of the wxx MI355X backend on BASELINE.json config 2 (1 GPU).

One step = one pass over config 2's standalone workload with inputs already
resident in HBM:
  * fp32 GEMM C = A @ B at M=N=K in {1024, 2048, 4096} and the two Linear
    shapes [8192x768]@[768x3072], [8192x3072]@[3072x768];
  * row softmax and LayerNorm on [8192 x 4096] fp32.

``value`` is the aggregate fp32 GEMM throughput of the step (total GEMM FLOP
/ total GEMM time).  Every kernel launch is bracketed by HIP events recorded
on the library's own stream; ``roofline`` reports the dominant kernel (the
4096^3 GEMM) against the 157.3 TFLOP/s fp32 matrix peak, and ``components``
reports each GEMM's TFLOP/s and the softmax / LayerNorm GB/s against 8 TB/s.
``cpu_baseline`` times the oracle's exact-order fp32 GEMM restatement
(oracle/csrc/gemm_ref.c, OpenMP on all host cores) on a bounded row sample of
the 4096^3 GEMM, on rank 0 at N=1 only.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

GEMMS = [
    ("gemm_1024", 1024, 1024, 1024),
    ("gemm_2048", 2048, 2048, 2048),
    ("gemm_4096", 4096, 4096, 4096),
    ("linear_8192x768x3072", 8192, 3072, 768),
    ("linear_8192x3072x768", 8192, 768, 3072),
]
ROWS, COLS = 8192, 4096


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


class Timer:
    """HIP events on the library stream; one slot pair per kernel call."""

    def __init__(self, lib):
        self.lib = lib
        self.samples = {}

    def run(self, name, fn):
        self.lib.call("wxx_timer_record", 0)
        fn()
        self.lib.call("wxx_timer_record", 1)
        ms = C.c_float(0.0)
        self.lib.call("wxx_timer_elapsed", 0, 1, C.byref(ms))
        self.samples.setdefault(name, []).append(ms.value)

    def avg(self, name):
        return float(np.mean(self.samples[name]))


def cpu_gemm_baseline(budget_s):
    """GFLOP/s of the oracle fp32 fma-chain GEMM on a row sample of 4096^3."""
    from oracle import gemm as og

    r = np.random.default_rng(0)
    n = 4096
    A = r.standard_normal((n, n), dtype=np.float32)
    B = r.standard_normal((n, n), dtype=np.float32)
    rows = 8
    og.matmul_add_fma(A, B, rows=(0, rows))  # load + warm
    total_rows, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        og.matmul_add_fma(A, B, rows=(0, rows))
        dt = time.perf_counter() - t0
        total_rows += rows
        elapsed += dt
        if dt < budget_s / 8:
            rows = min(n, rows * 2)
    flops = 2.0 * total_rows * n * n
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{total_rows} rows of the 4096x4096x4096 fp32 GEMM "
                  f"({elapsed:.1f} s), oracle/csrc/gemm_ref.c fma chain, OpenMP",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)

    from wxx_amd import functional as F
    from wxx_amd.backend import device, lib

    device.ensure_device()
    timer = Timer(lib)
    rng = np.random.default_rng(10)
    gemm_in = {}
    for name, M, N, K in GEMMS:
        gemm_in[name] = (F.from_numpy(rng.standard_normal((M, K), dtype=np.float32)),
                         F.from_numpy(rng.standard_normal((K, N), dtype=np.float32)))
    x = F.from_numpy(np.random.default_rng(20).standard_normal((ROWS, COLS), dtype=np.float32))
    gamma = F.from_numpy(np.ones(COLS, np.float32))
    beta = F.from_numpy(np.zeros(COLS, np.float32))
    keep = []

    def step():
        for name, *_ in GEMMS:
            a, b = gemm_in[name]
            timer.run(name, lambda: keep.append(F.matmul_add(a, b, None)))
        timer.run("softmax", lambda: keep.append(F.softmax(x, -1)))
        timer.run("layernorm", lambda: keep.append(F.meanvarnorm(x, gamma, beta, -1)))
        keep.clear()

    for _ in range(args.warmup):
        step()
    timer.samples.clear()
    lib.call("wxx_sync")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    lib.call("wxx_sync")
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    comps = {}
    gemm_flop = gemm_ms = 0.0
    for name, M, N, K in GEMMS:
        ms = timer.avg(name)
        flop = 2.0 * M * N * K
        gemm_flop += flop
        gemm_ms += ms
        comps[name] = {"tflops": flop / ms / 1e9, "ms": ms,
                       "frac_of_peak": flop / ms / 1e9 / PEAK_FP32_TFLOPS}
    sm_bytes = 2.0 * ROWS * COLS * 4
    ln_bytes = 2.0 * ROWS * COLS * 4 + 2 * COLS * 4 + 2 * ROWS * 4
    for name, nbytes in (("softmax", sm_bytes), ("layernorm", ln_bytes)):
        ms = timer.avg(name)
        comps[name] = {"gbs": nbytes / ms / 1e6, "ms": ms,
                       "frac_of_peak": nbytes / ms / 1e6 / PEAK_HBM_GBS}
    dom = comps["gemm_4096"]
    step_ms = sum(timer.avg(n) for n in timer.samples)
    out = {
        "metric": "GPT2 train-step tokens/s; fp32 GEMM TFLOP/s; FFT+reduction GB/s (1 GPU)",
        "value": gemm_flop / gemm_ms / 1e9,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "wall_ms_per_step": wall_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) inputs (numpy default_rng(10)/(20)), resident in HBM",
        "config": {
            "workload": "BASELINE config 2: fp32 GEMM M=N=K 1024/2048/4096, "
                        "[8192x768]@[768x3072], [8192x3072]@[3072x768]; "
                        "row softmax and LayerNorm on [8192x4096]",
            "value_is": "aggregate fp32 GEMM TFLOP/s over the five GEMMs",
        },
        "roofline": {
            "kernel": "gemm_f32_mfma_kernel (4096x4096x4096)",
            "bound": "mfma",
            "achieved": dom["tflops"],
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dom["tflops"] / PEAK_FP32_TFLOPS,
            "traffic": None,
        },
        "components": comps,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_gemm_baseline(args.cpu_seconds)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
