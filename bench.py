"""Benchmark: quantized matmul through the HIP plugin's C ABI on one MI355X.

Headline (BASELINE.json metric, configs[1] at M=1): 4-bit group-64 decode
GEMV, K=4096, N=14336, fp16 x/scales/out.  One step = one quantized matmul
over one weight set.  Steps rotate over 16 distinct weight copies (528 MB,
more than twice the 256 MB Infinity Cache) so every step streams its weights
from HBM.  value = weight bytes (packed codes + scales + biases) per step x
steps / wall time of the timed steps, which replay a HIP graph of 16 steps
captured on the plugin's stream (launch overhead out of the loop, work not).

roofline: the GEMV kernel's average duration, from HIP event pairs around
individual launches on the plugin's stream, against the 8 TB/s HBM peak.
gemm: configs[3] (M=2048, K=4096, N=4096 and 14336, bf16) TFLOP/s against
the 2.5 PFLOP/s bf16 dense MFMA peak, when the GEMM path is available.
cpu_baseline: the oracle's OpenMP quantized GEMV (a port, not the
reference, which has no such op) on the host cores, same shape, ~10 s sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemm]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F16, BF16, F32 = 1, 2, 0


class Hip:
    """The few HIP runtime calls the benchmark needs, via ctypes."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so", mode=os.RTLD_NOW | os.RTLD_GLOBAL)

    def ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def event(self):
        e = ctypes.c_void_p()
        self.ck(self.L.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream):
        self.ck(self.L.hipEventRecord(e, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ck(self.L.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ck(self.L.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def capture(self, stream, fn):
        """Capture fn()'s launches on `stream` into an instantiated graph."""
        s = ctypes.c_void_p(stream)
        self.ck(self.L.hipStreamBeginCapture(s, 2), "hipStreamBeginCapture")  # relaxed
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            self.ck(self.L.hipStreamEndCapture(s, ctypes.byref(g)), "hipStreamEndCapture")
        ex = ctypes.c_void_p()
        self.ck(self.L.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return ex

    def launch(self, ex, stream):
        self.ck(self.L.hipGraphLaunch(ex, ctypes.c_void_p(stream)), "hipGraphLaunch")

    def sync(self, stream):
        self.ck(self.L.hipStreamSynchronize(ctypes.c_void_p(stream)), "hipStreamSynchronize")

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self.ck(self.L.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)), "hipMalloc")
        return p

    def free(self, p):
        self.ck(self.L.hipFree(p), "hipFree")


def calibrate_copy(hip, nbytes, reps=8):
    """A plain device-to-device copy of nbytes (ROCm runs it as a blit
    kernel), the known-size reference that scales the FETCH_SIZE/WRITE_SIZE
    counters of the profiled kernels to bytes."""
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.ck(hip.L.hipMemset(src, 0x5A, ctypes.c_size_t(nbytes)), "hipMemset")
    hip.ck(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    for _ in range(reps):
        hip.ck(hip.L.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3), "hipMemcpy D2D")
    hip.ck(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    hip.free(src)
    hip.free(dst)
    print(json.dumps({"calibrate_copy_bytes": nbytes, "reps": reps}), flush=True)


def make_weights(ctx, N, K, bits, gs, sb, copies, seed):
    """W ~ N(0, 0.02) on the host, quantized on the GPU by the plugin's
    op_quantize into `copies` distinct buffer sets."""
    from mlx_amd import runtime
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02)).reshape(N, K)
    wb = ctx.upload(w)
    del w
    G = K // gs
    sets = []
    for _ in range(copies):
        wq = ctx.alloc(N * K * bits // 8)
        s = ctx.alloc(N * G * runtime.esize(sb))
        b = ctx.alloc(N * G * runtime.esize(sb))
        ctx.quantize(wb, wq, s, b, N, K, gs, bits, F32, sb)
        sets.append((wq, s, b))
    ctx.sync()
    wb.free()
    return sets


def weight_bytes(N, K, bits, gs, sb):
    return N * K * bits // 8 + 2 * N * (K // gs) * (4 if sb == F32 else 2)


def bench_qmm(ctx, hip, M, K, N, bits, gs, xd, sbd, od, steps, warmup, kernel, copies=16, seed=1):
    from mlx_amd import runtime
    rng = np.random.default_rng(seed + 7)
    x32 = rng.standard_normal(M * K, dtype=np.float32).reshape(M, K)
    if xd == F16:
        xh = x32.astype(np.float16).view(np.uint16)
    elif xd == BF16:
        u = x32.view(np.uint32)
        xh = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    else:
        xh = x32
    xb = ctx.upload(xh)
    sets = make_weights(ctx, N, K, bits, gs, sbd, copies, seed)
    out = ctx.alloc(M * N * runtime.esize(od))
    stream = ctx.stream

    def step(i):
        wq, s, b = sets[i % copies]
        ctx.quantized_matmul(xb, wq, s, b, out, M, K, N, gs, bits, xd, sbd, od, kernel)

    for i in range(max(warmup, copies)):
        step(i)
    ctx.sync()

    # per-launch kernel duration: HIP event pairs around single launches
    n_ev = min(64, max(steps, copies))
    evs = [(hip.event(), hip.event()) for _ in range(n_ev)]
    for i, (a, b) in enumerate(evs):
        hip.record(a, stream)
        step(i)
        hip.record(b, stream)
    ctx.sync()
    kern_ms = [hip.elapsed_ms(a, b) for a, b in evs]
    kern_ms.sort()
    kern_avg = float(np.mean(kern_ms))

    # whole job: replay a graph of `copies` steps
    graph = hip.capture(stream, lambda: [step(i) for i in range(copies)])
    reps = max(1, steps // copies)
    hip.launch(graph, stream)
    hip.sync(stream)
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(reps):
        hip.launch(graph, stream)
    hip.record(e1, stream)
    hip.sync(stream)
    wall = time.perf_counter() - t0
    n_steps = reps * copies
    graph_ms = hip.elapsed_ms(e0, e1) / n_steps

    for t in [xb, out] + [b for st in sets for b in st]:
        t.free()
    # kernel_ms_avg: events around the graph replays on the plugin's stream,
    # per step (kernel time plus the small gaps between graph nodes);
    # single_ms_*: event pairs around single eager launches (adds event overhead)
    return {"steps": n_steps, "wall_s": wall, "ms_per_step": wall * 1e3 / n_steps,
            "kernel_ms_avg": graph_ms, "single_ms_avg": kern_avg,
            "single_ms_median": kern_ms[len(kern_ms) // 2]}


def cpu_baseline(M, K, N, bits, gs, budget_s=10.0):
    """The oracle's OpenMP GEMV on this host's cores, same shape, ~budget_s."""
    from oracle import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, F16, F16, seed=1)
    O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F16, F16, F16, variant="omp", threads=threads)
    n, t0 = 0, time.perf_counter()
    while True:
        O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F16, F16, F16, variant="omp",
                           threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    gbs = weight_bytes(N, K, bits, gs, F16) * n / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} calls of the OpenMP CPU quantized GEMV (oracle), M={M} K={K} N={N} "
                      f"{bits}-bit g{gs} f16, {el:.1f} s"}


GEMV_PROFILE = os.path.join(ROOT, "profiles", "qgemv_m1_k4096_n14336_4bit_g64_f16.md")


def profiled_traffic(path):
    """HBM bytes per launch of the headline kernel: FETCH_SIZE + WRITE_SIZE
    from two rocprofv3 --pmc runs of this script, each scaled by the same
    counter's reading for a plain copy of known size (the summary under
    profiles/ gives the commands and the factors).  None when absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


# (name, M, K, N, bits, group, x dtype, scale dtype, out dtype)
SWEEP = [
    ("c0", 1, 4096, 4096, 4, 64, F32, F32, F32),
    ("c1", 1, 4096, 14336, 4, 64, F16, F16, F16),
    ("c1", 4, 4096, 14336, 4, 64, F16, F16, F16),
    ("c1", 8, 4096, 14336, 4, 64, F16, F16, F16),
    ("c2", 32, 8192, 8192, 8, 128, BF16, BF16, BF16),
    ("c3", 2048, 4096, 4096, 4, 64, BF16, BF16, BF16),
    ("c3", 2048, 4096, 14336, 4, 64, BF16, BF16, BF16),
    ("c4", 1, 4096, 11008, 3, 64, F16, F16, F16),
    ("c4", 1, 4096, 11008, 6, 64, F16, F16, F16),
    ("c4", 64, 4096, 11008, 3, 64, F16, F16, F16),
    ("c4", 64, 4096, 11008, 6, 64, F16, F16, F16),
]


def sweep(ctx, hip, steps):
    """One line per config: kernel AUTO picks, graph-replay time per launch,
    weight GB/s and TFLOP/s with their roofline fractions."""
    from mlx_amd import abi
    names = {abi.KERNEL_GEMV: "gemv", abi.KERNEL_GEMM: "gemm"}
    for name, M, K, N, bits, gs, xd, sbd, od in SWEEP:
        kern = ctx.select_kernel(M, K, N, gs, bits, xd, sbd)
        copies = 4 if M >= 256 else 16
        r = bench_qmm(ctx, hip, M, K, N, bits, gs, xd, sbd, od, steps, 8, abi.KERNEL_AUTO, copies=copies)
        t = r["kernel_ms_avg"] * 1e-3
        wb = weight_bytes(N, K, bits, gs, sbd)
        flops = 2.0 * M * N * K
        print(json.dumps({"config": name, "M": M, "K": K, "N": N, "bits": bits, "group_size": gs,
                          "kernel": names.get(kern, str(kern)), "us": round(t * 1e6, 3),
                          "weight_GBs": round(wb / t / 1e9, 1), "hbm_frac": round(wb / t / 1e9 / HBM_PEAK_GBS, 4),
                          "tflops": round(flops / t / 1e12, 2),
                          "mfma_frac": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4)}), flush=True)


def decode_legs(ctx, hip, K, N, bits, gs, steps):
    """configs[1] at M=4 and M=8: same weight bytes as M=1, 4x / 8x the math."""
    from mlx_amd import abi
    out = {}
    wb = weight_bytes(N, K, bits, gs, F16)
    for m in (4, 8):
        r = bench_qmm(ctx, hip, m, K, N, bits, gs, F16, F16, F16, min(steps, 1024), 16, abi.KERNEL_AUTO)
        t = r["kernel_ms_avg"] * 1e-3
        out[f"M{m}"] = {"kernel_us_avg": round(t * 1e6, 3), "weight_GBs": round(wb / t / 1e9, 1),
                        "hbm_frac": round(wb / t / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the headline line, one JSON line per BASELINE config")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the configs[1] M=4 and M=8 decode legs (for profiling)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a device-to-device copy of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy(Hip(), args.calibrate_copy)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the plugin path is single-device; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    from mlx_amd import abi, runtime
    hip = Hip()
    ctx = runtime.Context(0)
    if args.sweep:
        sweep(ctx, hip, min(args.steps, 256))
        ctx.close()
        return

    M, K, N, bits, gs = 1, 4096, 14336, 4, 64
    if args.decode_only:
        print(json.dumps({"decode_m4_m8": decode_legs(ctx, hip, K, N, bits, gs, args.steps)}), flush=True)
        ctx.close()
        return
    r = bench_qmm(ctx, hip, M, K, N, bits, gs, F16, F16, F16, args.steps, args.warmup,
                  abi.KERNEL_AUTO)
    wb = weight_bytes(N, K, bits, gs, F16)
    value = wb * r["steps"] / r["wall_s"] / 1e9
    achieved = wb / (r["kernel_ms_avg"] * 1e-3) / 1e9
    line = {
        "metric": "weight GB/s (%HBM peak) at M=1 & TFLOP/s (%MFMA peak) at M=2048, 4-bit",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: x~N(0,1) f16; W~N(0,0.02) quantized on the GPU (4-bit, group 64, "
                "f16 scales/biases); 16 rotated weight copies",
        "config": {"workload": "configs[1] decode GEMV M=1", "M": M, "K": K, "N": N, "bits": bits,
                   "group_size": gs, "kernel": "gemv", "hbm_pct": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(GEMV_PROFILE),
                     "kernel": "qgemv_stream_kernel", "kernel_us_avg": round(r["kernel_ms_avg"] * 1e3, 3),
                     "kernel_us_single_launch": round(r["single_ms_avg"] * 1e3, 3),
                     "algorithmic_bytes": wb},
    }
    line["decode_m4_m8"] = decode_legs(ctx, hip, K, N, bits, gs, args.steps)
    if not args.no_gemm:
        gemm = {}
        for n in (4096, 14336):
            if ctx.select_kernel(2048, 4096, n, 64, 4, BF16) != abi.KERNEL_GEMM:
                break
            rg = bench_qmm(ctx, hip, 2048, 4096, n, 4, 64, BF16, BF16, BF16, min(args.steps, 256),
                           8, abi.KERNEL_AUTO, copies=4)
            flops = 2.0 * 2048 * 4096 * n
            tf = flops / (rg["kernel_ms_avg"] * 1e-3) / 1e12
            gemm[f"N{n}"] = {"tflops": round(tf, 2), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                             "kernel_us_avg": round(rg["kernel_ms_avg"] * 1e3, 2),
                             "wall_tflops": round(flops * rg["steps"] / rg["wall_s"] / 1e12, 2)}
        line["gemm_m2048"] = gemm or None
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(M, K, N, bits, gs)
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
