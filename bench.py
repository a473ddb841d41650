"""Benchmark of the wxx MI355X backend on BASELINE.json config 2 (1 GPU).

One step = one pass over config 2's standalone workload with inputs already
resident in HBM:
  * fp32 GEMM C = A @ B at M=N=K in {1024, 2048, 4096} and the two Linear
    shapes [8192x768]@[768x3072], [8192x3072]@[3072x768];
  * row softmax and LayerNorm on [8192 x 4096] fp32.

``value`` is the aggregate fp32 GEMM throughput of the step (total GEMM FLOP
/ total GEMM time).  Each kernel is timed over ``--reps`` back-to-back
launches between one pair of HIP events recorded on the library's own stream
(the stream every kernel runs on), with outputs preallocated and the C ABI
called directly, so the average is the kernel's own duration and agrees with
``rocprofv3 --kernel-trace``.  ``roofline`` reports the dominant kernel (the
4096^3 GEMM) against the 157.3 TFLOP/s fp32 matrix peak; ``components``
reports every kernel of the step, and ``extra`` the HBM-bound kernels of the
other configs measured on the same box (config 4's standalone batched real
FFT / inverse FFT on [2048 x 16384], a row sum over [8192 x 4096]) and a
256 MiB device-to-device copy as the achievable-bandwidth reference; and
the train steps of configs 1 and 5 (GPT-2), 3 (ResNet18) and 4 (Hyena):
forward, CCE loss, backward, clip_grad_norm_, AdamW, LR schedule, in tokens/s
or images/s, timed on the host clock between device synchronisations.
``gpt2_train_step`` reports the config-5 train step (the metric's first
quantity, on the north star's target config) with its model-FLOP rate;
``train_steps`` holds all four model configs.  ``cpu_baseline`` times the
oracle's exact-order fp32 GEMM restatement (oracle/csrc/gemm_ref.c, OpenMP on
the host cores) on a bounded row sample of the 4096^3 GEMM, and under
``components`` the oracle's numpy softmax, LayerNorm, rfft and config-1
train step on bounded samples, on rank 0 at N=1 only.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-cpu]
                       [--no-train] [--only NAME]
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
FFT_ROWS, FFT_N = 2048, 16384
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemm_4096.json")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--reps", type=int, default=0,
                   help="launches per timed kernel per step (0: about 2 ms of work each)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default=None, help="run only this component (profiling)")
    p.add_argument("--no-train", action="store_true", help="skip the train-step extras")
    p.add_argument("--graph-only", action="store_true",
                   help="with --only TRAIN_CONFIG: time only the step-graph replays")
    return p.parse_args()


def cpu_gemm_baseline(budget_s):
    """TFLOP/s of the oracle fp32 fma-chain GEMM on a row sample of 4096^3."""
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


def _cpu_rate(fn, budget_s):
    """(calls, seconds) of repeating ``fn`` for about ``budget_s`` (one
    untimed warm call first)."""
    fn()
    calls, elapsed = 0, 0.0
    while elapsed < budget_s or calls == 0:
        t0 = time.perf_counter()
        fn()
        elapsed += time.perf_counter() - t0
        calls += 1
    return calls, elapsed


def cpu_component_baselines(budget_s):
    """The oracle's numpy restatements of the HBM-bound config-2/4 kernels and
    of the config-1 train step, timed on the host cores (numpy float64 math;
    BLAS threads for the train step)."""
    from oracle import activations as oa
    from oracle import fft as of
    from oracle import models as om
    from oracle import norms as on

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rows = ROWS // 16
    r = np.random.default_rng(20)
    x = r.standard_normal((rows, COLS), dtype=np.float32)
    g, b = np.ones(COLS, np.float32), np.zeros(COLS, np.float32)
    out = {}
    n, t = _cpu_rate(lambda: oa.softmax(x, -1), budget_s)
    out["softmax"] = {"gbs": n * 2.0 * rows * COLS * 4 / t / 1e9, "cores": 1,
                      "sample": f"{n} x [{rows}x4096] row softmax (1/16 of config 2's rows), "
                                "oracle/activations.py (numpy, float64)"}
    n, t = _cpu_rate(lambda: on.meanvarnorm(x, g, b, -1), budget_s)
    out["layernorm"] = {"gbs": n * 2.0 * rows * COLS * 4 / t / 1e9, "cores": 1,
                        "sample": f"{n} x [{rows}x4096] LayerNorm (1/16 of config 2's rows), "
                                  "oracle/norms.py (numpy, float64)"}
    fx = np.random.default_rng(41).standard_normal((FFT_ROWS // 8, FFT_N), dtype=np.float32)
    nb = FFT_N // 2 + 1
    n, t = _cpu_rate(lambda: of.rfft(fx, FFT_N), budget_s)
    out["rfft"] = {"gbs": n * (FFT_ROWS // 8) * (FFT_N * 4.0 + nb * 8) / t / 1e9, "cores": 1,
                   "sample": f"{n} x [256x16384] rfft (1/8 of config 4's rows), oracle/fft.py "
                             "(numpy pocketfft, float64)"}
    V, D, H, L, B, S = 1024, 256, 8, 6, 4, 128
    rp = np.random.default_rng(1234)
    P = {"tok_emb.weight": rp.normal(0, 0.02, (V, D)), "pos_emb.weight": rp.normal(0, 0.02, (256, D)),
         "ln_f.weightg": np.ones(D), "ln_f.weightb": np.zeros(D)}
    for i in range(L):
        p = f"blocks.{i}."
        for nm in ("q", "k", "v", "out"):
            P[p + f"attn.{nm}.weight"] = rp.normal(0, 0.02, (D, D))
        P[p + "mlp.0.weight"], P[p + "mlp.0.bias"] = rp.normal(0, 0.02, (D, 4 * D)), np.zeros(4 * D)
        P[p + "mlp.2.weight"], P[p + "mlp.2.bias"] = rp.normal(0, 0.02, (4 * D, D)), np.zeros(D)
        for ln in ("ln1", "ln2"):
            P[p + f"{ln}.weightg"], P[p + f"{ln}.weightb"] = np.ones(D), np.zeros(D)
    ids = np.random.default_rng(0).integers(0, V, (B, S))
    tg = np.random.default_rng(1).integers(0, V, (B, S))
    n, t = _cpu_rate(lambda: om.gpt2_loss_and_grads(P, ids, tg, H, L), budget_s)
    out["gpt2_train_config1"] = {
        "tokens_per_s": n * B * S / t, "cores": threads,
        "sample": f"{n} forward+backward passes of GPT2(1024, 256, 8, 6) on 4 x 128 tokens, "
                  "oracle/models.py (numpy float64, BLAS threads)"}
    return out


class Kernels:
    """Preallocated operands and one zero-argument launcher per component."""

    def __init__(self, lib):
        from wxx_amd import functional as F

        self.F = F
        self.keep = []
        self.launch = {}
        self.work = {}  # name -> (amount, unit kind "flop" | "byte")
        rng = np.random.default_rng(10)
        for name, M, N, K in GEMMS:
            a = self._up(rng.standard_normal((M, K), dtype=np.float32))
            b = self._up(rng.standard_normal((K, N), dtype=np.float32))
            c = self._empty((M, N))
            self.launch[name] = self._gemm(lib, a, b, c, M, N, K)
            self.work[name] = (2.0 * M * N * K, "flop")
        x = self._up(np.random.default_rng(20).standard_normal((ROWS, COLS), dtype=np.float32))
        y = self._empty((ROWS, COLS))
        g = self._up(np.ones(COLS, np.float32))
        bt = self._up(np.zeros(COLS, np.float32))
        mu, istd = self._empty((ROWS,)), self._empty((ROWS,))
        P = C.c_void_p
        self.launch["softmax"] = lambda: lib.call("wxx_softmax", P(x.data_ptr()),
                                                  P(y.data_ptr()), 1 * ROWS, COLS, 1)
        self.work["softmax"] = (2.0 * ROWS * COLS * 4, "byte")
        self.launch["layernorm"] = lambda: lib.call(
            "wxx_meanvarnorm", P(x.data_ptr()), P(g.data_ptr()), P(bt.data_ptr()),
            P(y.data_ptr()), P(mu.data_ptr()), P(istd.data_ptr()), ROWS, COLS, 1,
            C.c_float(1e-5), 0)
        self.work["layernorm"] = (2.0 * ROWS * COLS * 4 + 2 * COLS * 4 + 2 * ROWS * 4, "byte")
        s = self._empty((ROWS,))
        self.launch["row_sum"] = lambda: lib.call("wxx_reduce", P(x.data_ptr()),
                                                  P(s.data_ptr()), ROWS, COLS, 1, 0)
        self.work["row_sum"] = (ROWS * COLS * 4.0 + ROWS * 4, "byte")
        fx = self._up(np.random.default_rng(41).standard_normal((FFT_ROWS, FFT_N),
                                                               dtype=np.float32))
        nb = FFT_N // 2 + 1
        fX = self._empty((FFT_ROWS, nb), dtype="c64")
        fy = self._empty((FFT_ROWS, FFT_N))
        self.launch["rfft_2048x16384"] = lambda: lib.call(
            "wxx_rfft", P(fx.data_ptr()), P(fX.data_ptr()), FFT_ROWS, FFT_N, FFT_N)
        self.work["rfft_2048x16384"] = (FFT_ROWS * (FFT_N * 4.0 + nb * 8), "byte")
        self.launch["irfft_2048x16384"] = lambda: lib.call(
            "wxx_irfft", P(fX.data_ptr()), P(fy.data_ptr()), FFT_ROWS, nb, FFT_N)
        self.work["irfft_2048x16384"] = (FFT_ROWS * (FFT_N * 4.0 + nb * 8), "byte")
        # device-to-device copy of 256 MiB: the achievable-bandwidth reference and
        # the calibration kernel for the HBM byte counters
        cb = 256 << 20
        csrc, cdst = self._empty((cb // 4,)), self._empty((cb // 4,))
        self.launch["copy_256MiB"] = lambda: lib.call("wxx_d2d", P(cdst.data_ptr()),
                                                      P(csrc.data_ptr()), cb)
        self.work["copy_256MiB"] = (2.0 * cb, "byte")

    def _up(self, a):
        t = self.F.from_numpy(a)
        self.keep.append(t)
        return t

    def _empty(self, shape, dtype="f32"):
        from wxx_amd.functional._common import empty

        t = empty(shape, dtype=dtype)
        self.keep.append(t)
        return t

    @staticmethod
    def _gemm(lib, a, b, c, M, N, K):
        P = C.c_void_p
        pa, pb, pc = P(a.data_ptr()), P(b.data_ptr()), P(c.data_ptr())
        return lambda: lib.call("wxx_matmul_add", pa, pb, None, pc, M, N, K, 1, 0, 0, 0, 0, 0, 0,
                                0)


# BASELINE train-step configs: GPT-2 (1, 5), ResNet18 (3), Hyena (4); dropout 0.
TRAIN_CONFIGS = {
    "gpt2_train_config1": dict(kind="gpt2", V=1024, D=256, H=8, L=6, B=4, S=128, max_len=256,
                               flop=1.651e10),
    "resnet18_train_config3": dict(kind="resnet18", classes=10, B=128, HW=32),
    "hyena_train_config4": dict(kind="hyena", V=1024, D=256, L=6, order=4, B=8, S=8192),
    "gpt2_train_config5": dict(kind="gpt2", V=50304, D=768, H=12, L=12, B=8, S=1024,
                               max_len=1024, flop=7.001e12),
}


def _train_setup(wxx, c, r):
    """Model, optimizer, inputs and a loss closure for one BASELINE train config
    (random-init weights, synthetic inputs of the config's shape)."""
    F = wxx.functional
    lossf = wxx.nn.CCELoss()
    if c["kind"] == "gpt2":
        m = wxx.nn.GPT2(c["V"], c["D"], c["H"], c["L"], max_len=c["max_len"], dropout=0.0)
        x = F.from_numpy(r.integers(0, c["V"], (c["B"], c["S"])), np.uint32)
        y = F.from_numpy(r.integers(0, c["V"], (c["B"] * c["S"],)), np.uint32)
        loss = lambda: lossf(m(x).reshape((c["B"] * c["S"], c["V"])), y)  # noqa: E731
        units, unit = c["B"] * c["S"], "tokens"
        desc = (f"GPT2(vocab {c['V']}, d {c['D']}, heads {c['H']}, layers {c['L']}), "
                f"batch {c['B']} x seq {c['S']}, dropout 0")
    elif c["kind"] == "resnet18":
        m = wxx.nn.ResNet18(num_classes=c["classes"])
        x = F.from_numpy(r.standard_normal((c["B"], 3, c["HW"], c["HW"]), dtype=np.float32))
        y = F.from_numpy(r.integers(0, c["classes"], (c["B"],)), np.uint32)
        loss = lambda: lossf(m(x), y)  # noqa: E731
        units, unit = c["B"], "images"
        desc = f"ResNet18(num_classes {c['classes']}), batch {c['B']} x 3x{c['HW']}x{c['HW']}"
    else:
        m = wxx.nn.Hyena(c["V"], d_model=c["D"], n_layers=c["L"], order=c["order"])
        x = F.from_numpy(r.integers(0, c["V"], (c["B"], c["S"])), np.uint32)
        y = F.from_numpy(r.integers(0, c["V"], (c["B"] * c["S"],)), np.uint32)
        loss = lambda: lossf(m(x).reshape((c["B"] * c["S"], c["V"])), y)  # noqa: E731
        units, unit = c["B"] * c["S"], "tokens"
        desc = (f"Hyena(vocab {c['V']}, d {c['D']}, layers {c['L']}, order {c['order']}), "
                f"batch {c['B']} x seq {c['S']}")
    return m, loss, units, unit, desc


def train_step(lib, name, steps, warmup, graph_steps=None, eager=True):
    """Full train step: forward, CCELoss, backward, clip_grad_norm_(1.0), AdamW,
    WarmupCosineLR (README.md:50-51 schedule), zero_grad.  Timed with the host
    clock around ``steps`` steps between device synchronisations, first run
    eagerly (every op dispatched from Python), then recorded once as a step
    graph and replayed ``graph_steps`` times (the same steps continue).  With
    ``eager`` False only the warm-up runs eagerly (profiling the replays)."""
    import wxx_amd as wxx

    c = TRAIN_CONFIGS[name]
    m, lossfn, units, unit, desc = _train_setup(wxx, c, np.random.default_rng(50))
    opt = wxx.nn.AdamW(m.parameters(), lr=1e-3)
    sched = wxx.nn.WarmupCosineLR(opt, warmup_steps=100, total_steps=5000, min_lr=1e-5)

    def step():
        loss = lossfn()
        loss.backward()
        wxx.nn.clip_grad_norm_(m.parameters(), 1.0)
        opt.step()
        sched.step()
        opt.zero_grad()
        return loss

    for _ in range(max(warmup, 1)):
        loss = step()
    lib.call("wxx_sync")
    out = {"model": desc}
    if eager:
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        lib.call("wxx_sync")
        dt = (time.perf_counter() - t0) / steps
        out.update({f"{unit}_per_s": units / dt, "ms": dt * 1e3, "steps_timed": steps,
                    "loss": float(loss.numpy().reshape(-1)[0])})
        if "flop" in c:
            out["tflops"] = c["flop"] / dt / 1e12
            out["frac_of_peak"] = out["tflops"] / PEAK_FP32_TFLOPS
    graph_steps = steps if graph_steps is None else graph_steps
    if graph_steps:
        try:
            g = wxx.StepGraph(step).capture()
        except Exception as e:  # reported, not fatal: the eager figure stands
            out["graph"] = {"error": f"{type(e).__name__}: {e}"}
            return out
        g.replay()  # first launch of a new graph uploads its code objects
        lib.call("wxx_sync")
        t0 = time.perf_counter()
        for _ in range(graph_steps):
            loss = g.replay()
        lib.call("wxx_sync")
        gdt = (time.perf_counter() - t0) / graph_steps
        out["graph"] = {f"{unit}_per_s": units / gdt, "ms": gdt * 1e3,
                        "steps_timed": graph_steps, "nodes": g.nodes,
                        "loss": float(loss.numpy().reshape(-1)[0])}
        if "flop" in c:
            out["graph"]["tflops"] = c["flop"] / gdt / 1e12
            out["graph"]["frac_of_peak"] = out["graph"]["tflops"] / PEAK_FP32_TFLOPS
        g.close()
    return out


STEP = [n for n, *_ in GEMMS] + ["softmax", "layernorm"]
EXTRA = ["row_sum", "rfft_2048x16384", "irfft_2048x16384", "copy_256MiB"]


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(every box in this build has a single MI355X)", file=sys.stderr)
        sys.exit(2)

    from wxx_amd.backend import device, lib

    device.ensure_device()
    ks = Kernels(lib)
    names = STEP + EXTRA
    if args.only in TRAIN_CONFIGS:
        print(json.dumps({"only": args.only,
                          "component": train_step(lib, args.only, args.steps, args.warmup,
                                                  eager=not args.graph_only)}))
        return
    if args.only:
        names = [args.only]

    def reps_for(name):
        if args.reps:
            return args.reps
        amount, kind = ks.work[name]
        est_ms = amount / (80e9 if kind == "flop" else 4e9)  # rough 80 TF/s, 4 TB/s, per ms
        return int(min(200, max(3, round(2.0 / max(est_ms, 1e-3)))))

    reps = {n: reps_for(n) for n in names}
    samples = {n: [] for n in names}
    ms = C.c_float(0.0)

    def run_step(record):
        for n in names:
            lib.call("wxx_timer_record", 0)
            for _ in range(reps[n]):
                ks.launch[n]()
            lib.call("wxx_timer_record", 1)
            lib.call("wxx_timer_elapsed", 0, 1, C.byref(ms))
            if record:
                samples[n].append(ms.value / reps[n])

    for _ in range(args.warmup):
        run_step(False)
    lib.call("wxx_sync")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(True)
    lib.call("wxx_sync")
    wall_s = time.perf_counter() - t0

    comps = {}
    for n in names:
        t = float(np.median(samples[n]))
        amount, kind = ks.work[n]
        if kind == "flop":
            rate = amount / t / 1e9
            comps[n] = {"tflops": rate, "ms": t, "frac_of_peak": rate / PEAK_FP32_TFLOPS,
                        "launches_timed": reps[n] * args.steps}
        else:
            rate = amount / t / 1e6
            comps[n] = {"gbs": rate, "ms": t, "frac_of_peak": rate / PEAK_HBM_GBS,
                        "launches_timed": reps[n] * args.steps}
    if args.only:
        print(json.dumps({"only": args.only, "component": comps[args.only]}))
        return

    gemm_flop = sum(ks.work[n][0] for n, *_ in GEMMS)
    gemm_ms = sum(comps[n]["ms"] for n, *_ in GEMMS)
    step_ms = sum(comps[n]["ms"] for n in STEP)
    dom = comps["gemm_4096"]
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    out = {
        "metric": "GPT2 train-step tokens/s; fp32 GEMM TFLOP/s; FFT+reduction GB/s (1 GPU)",
        "value": gemm_flop / gemm_ms / 1e9,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) inputs (numpy default_rng(10)/(20)/(41)), resident in HBM",
        "config": {
            "workload": "BASELINE config 2: fp32 GEMM M=N=K 1024/2048/4096, "
                        "[8192x768]@[768x3072], [8192x3072]@[3072x768]; "
                        "row softmax and LayerNorm on [8192x4096]",
            "value_is": "aggregate fp32 GEMM TFLOP/s over the five GEMMs of the step",
            "timing": "per kernel: median over steps of (HIP-event time of R back-to-back "
                      "launches on the library stream) / R; the rocprofv3 per-dispatch trace "
                      "of the same command is in profiles/kernels_bench_config2.md",
        },
        "roofline": {
            "kernel": "gemm_f32_dtl_kernel<false,false> (4096x4096x4096)",
            "bound": "mfma",
            "achieved": dom["tflops"],
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dom["tflops"] / PEAK_FP32_TFLOPS,
            "traffic": traffic,
        },
        "components": {n: comps[n] for n in STEP},
        "extra": {n: comps[n] for n in EXTRA},
        "wall_s": wall_s,
    }
    if not args.no_train:
        out["train_steps"] = {name: train_step(lib, name, steps=5, warmup=2)
                              for name in TRAIN_CONFIGS}
        c5 = out["train_steps"]["gpt2_train_config5"]
        # the metric's first quantity, on the north star's target config
        out["gpt2_train_step"] = {
            "tokens_per_s": c5["tokens_per_s"], "ms_per_step": c5["ms"],
            "model_tflops": c5["tflops"], "frac_of_fp32_peak": c5["frac_of_peak"],
            "steps_timed": c5["steps_timed"], "loss": c5["loss"],
            "config": c5["model"] + "; forward, CCELoss, backward, clip_grad_norm_(1.0), "
                      "AdamW, WarmupCosineLR",
            "model_flop_per_step": TRAIN_CONFIGS["gpt2_train_config5"]["flop"],
            "graph_tokens_per_s": c5.get("graph", {}).get("tokens_per_s"),
            "graph_ms_per_step": c5.get("graph", {}).get("ms"),
            "graph_frac_of_fp32_peak": c5.get("graph", {}).get("frac_of_peak"),
            "timing": "host clock around 5 steps between device synchronisations; graph_*: "
                      "the same steps recorded once as a step graph and replayed",
            "profile": "profiles/gpt2_config5_train_step.md"}
    if not args.no_cpu:
        base = cpu_gemm_baseline(args.cpu_seconds)
        base["components"] = cpu_component_baselines(args.cpu_seconds / 4)
        out["cpu_baseline"] = base
    print(json.dumps(out))


if __name__ == "__main__":
    main()
