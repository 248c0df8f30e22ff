"""Benchmark: quantized matmul through the HIP plugin's C ABI on one MI355X.

Headline (BASELINE.json metric, configs[1] at M=1): 4-bit group-64 decode
GEMV, K=4096, N=14336, fp16 x/scales/out.  One step = one quantized matmul
over one weight set.  Steps rotate over 16 distinct weight copies (528 MB,
more than twice the 256 MB Infinity Cache) so every step streams its weights
from HBM.  The timed region is exactly --steps launches issued back to back
on the plugin's stream, bracketed by a synchronize on both sides:
value = weight bytes (packed codes + scales + biases) x steps / host wall time
of the region.

roofline: HIP events on the plugin's stream around the same timed region give
the average launch duration (kernel plus the gap to the next launch);
achieved = algorithmic weight bytes / that duration, against 8 TB/s.  The
same launches replayed as 16-launch HIP graphs are reported beside it.
ceiling: an empty kernel and a plain read of the same 33 030 144 bytes (the
fastest single-launch read pattern measured), timed the same way: what one
launch of this size can show at all on this box.
decode_m4_m8: configs[1] at M=4 and M=8.  gemm_m2048: configs[3] (M=2048,
K=4096, N=4096 and 14336, bf16) TFLOP/s against the 2.5 PFLOP/s bf16 dense
MFMA peak.
cpu_baseline: the oracle's OpenMP quantized GEMV (a port: the reference has
no quantized op) on all of this process's host cores and on one, plus the
reference's own composition (host dequantize, then the reference CPU
backend's op_matmul_f32 built from its source into oracle/_ref/); the same
leg also uses the oracle as the checker of the GPU outputs (parity:
max|d|/max|y| of c1, c2 and c3).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemm]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

# Kernel arguments in device memory (a HIP runtime setting, read when the
# runtime initializes, so before anything here loads it): each launch's
# waves then read their arguments from HBM rather than across PCIe from host
# memory.  Alternated on one box (bench legs, HIP events per launch): c1
# 8.65-8.72 -> 7.81-7.92 us, the plain 33 MB read 7.14-7.20 -> 6.18-6.21, c0
# 6.8-7.0 -> 4.95-5.0, decode M = 4 10.2-10.3 -> 9.19-9.25; graph replays
# unchanged (7.50 / 7.47 us at c1).  A value already in the environment is
# kept; the line reports the one in effect.
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F16, BF16, F32 = 1, 2, 0
COPIES = 16


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

    def memset(self, p, value, nbytes):
        self.ck(self.L.hipMemset(p, value, ctypes.c_size_t(nbytes)), "hipMemset")

    def free(self, p):
        self.ck(self.L.hipFree(p), "hipFree")


# Every leg first runs its own launches for at least this long (and at least
# --warmup launches): a leg that follows seconds of host-side set-up (weight
# generation, upload) otherwise starts on a GPU whose clocks are still
# ramping, which a handful of warm-up launches does not cover.
WARM_S = 0.3


def warm(hip, stream, step, launches, warm_s=WARM_S):
    """At least `launches` launches and at least warm_s seconds of them
    (batches of launches, a synchronize after each, until both hold)."""
    t0, n = time.perf_counter(), 0
    while True:
        for _ in range(max(1, min(launches, 64))):
            step(n)
            n += 1
        hip.sync(stream)
        if n >= launches and time.perf_counter() - t0 >= warm_s:
            return n


def per_launch_us(hip, stream, step, steps):
    """The same launches again with an event before each and one after the
    last: the median and spread of the per-launch durations (kernel plus the
    gap to the next launch), and the first three (a clock ramp shows there)."""
    ev = [hip.event() for _ in range(steps + 1)]
    hip.sync(stream)
    for i in range(steps):
        hip.record(ev[i], stream)
        step(i)
    hip.record(ev[steps], stream)
    hip.sync(stream)
    d = np.array([hip.elapsed_ms(ev[i], ev[i + 1]) * 1e3 for i in range(steps)])
    for e in ev:
        hip.L.hipEventDestroy(e)
    return {"median": round(float(np.median(d)), 3), "p10": round(float(np.percentile(d, 10)), 3),
            "p90": round(float(np.percentile(d, 90)), 3), "first": [round(float(v), 3) for v in d[:3]]}


def time_launches(hip, stream, step, steps, warmup, loop=None):
    """Warm-up (warm(): at least `warmup` launches and WARM_S seconds), then
    exactly `steps` launches back to back on `stream` between a synchronize
    on each side; returns host wall time of the region and the HIP-event
    time per launch, then the per-launch durations of the same launches run
    once more (per_launch_us).  step(i) enqueues launch i (rotating over the
    weight copies itself); loop(first, n), where given, enqueues launches
    first .. first + n - 1 from C and issues the timed ones."""
    warm(hip, stream, step, warmup)
    e0, e1 = hip.event(), hip.event()
    hip.sync(stream)
    t0 = time.perf_counter()
    hip.record(e0, stream)
    if loop is not None:
        loop(0, steps)
    else:
        for i in range(steps):
            step(i)
    hip.record(e1, stream)
    hip.sync(stream)
    wall = time.perf_counter() - t0
    r = {"wall_s": wall, "event_ms_per_launch": hip.elapsed_ms(e0, e1) / steps}
    r["per_launch_us"] = per_launch_us(hip, stream, step, steps)
    return r


def time_graph(hip, stream, step, reps=32):
    """The same launches replayed as COPIES-launch graphs: per launch."""
    graph = hip.capture(stream, lambda: [step(i) for i in range(COPIES)])
    hip.launch(graph, stream)
    hip.sync(stream)
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(reps):
        hip.launch(graph, stream)
    hip.record(e1, stream)
    hip.sync(stream)
    return hip.elapsed_ms(e0, e1) / (reps * COPIES)


def calibrate_copy(hip, nbytes, reps=8):
    """A plain device-to-device copy of nbytes (ROCm runs it as a blit
    kernel), the known-size reference that scales the FETCH_SIZE/WRITE_SIZE
    counters of the profiled kernels to bytes."""
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.memset(src, 0x5A, nbytes)
    hip.ck(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    for _ in range(reps):
        hip.ck(hip.L.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3), "hipMemcpy D2D")
    hip.ck(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    hip.free(src)
    hip.free(dst)
    print(json.dumps({"calibrate_copy_bytes": nbytes, "reps": reps}), flush=True)


# ---- synthetic inputs: the fixtures' portable generator -------------------
# x ~ N(0, 1) from stream 4 seed + 1, W ~ N(0, 0.02) from stream 4 seed + 2
# and, for configs[4], 1 % of W's entries scaled by 20 (chosen by a stable
# sort of the u32 stream 4 seed + 3): the tensors whose SHA-256 digests
# tests/golden/digests.json holds (each leg's copy-0 weights are checked
# against them; digest_match in the line).
DIGESTS = os.path.join(ROOT, "tests", "golden", "digests.json")
_W_CACHE = {}


def rng_normal(n, seed, std=1.0):
    L = ceiling_lib()
    out = np.empty(n, dtype=np.float32)
    L.lux_bench_rng_normal_f32(out.ctypes.data, n, seed, 0.0, std)
    return out


def w_host(N, K, seed, outliers):
    key = (N, K, seed, outliers)
    if key not in _W_CACHE:
        _W_CACHE.clear()
        w = rng_normal(N * K, seed * 4 + 2, 0.02)
        if outliers:
            L = ceiling_lib()
            u = np.empty(N * K, dtype=np.uint32)
            L.lux_bench_rng_u32(u.ctypes.data, N * K, seed * 4 + 3)
            w[u.argsort(kind="stable")[:int(round(0.01 * N * K))]] *= np.float32(20.0)
        _W_CACHE[key] = w.reshape(N, K)
    return _W_CACHE[key]


def make_weights(ctx, N, K, bits, gs, sb, copies, seed, outliers=False):
    """W on the host (the generator above), quantized on the GPU by the
    plugin's op_quantize into `copies` distinct buffer sets."""
    from mlx_amd import runtime
    wb = ctx.upload(w_host(N, K, seed, outliers))
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


def digest_match(K, N, bits, gs, sb, seed, outliers, w_q, s, b):
    """Whether copy 0's quantized weights hash to the committed digests of
    the config with this shape (None where no digest covers it)."""
    import hashlib
    try:
        with open(DIGESTS) as f:
            table = json.load(f)
    except OSError:
        return None
    for d in table.values():
        if (d["shape"][1:] == [K, N] and d["bits"] == bits and d["group_size"] == gs and d["sb_dtype"] == sb
                and d["seed"] == seed and bool(d.get("outlier_frac")) == outliers):
            got = {n: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
                   for n, a in (("w_q", w_q), ("scales", s), ("biases", b))}
            return all(got[n] == d["sha256"][n] for n in got)
    return None


def weight_bytes(N, K, bits, gs, sb):
    return N * K * bits // 8 + 2 * N * (K // gs) * (4 if sb == F32 else 2)


def x_host(M, K, xd, seed):
    x32 = rng_normal(M * K, seed * 4 + 1).reshape(M, K)
    if xd == F16:
        return x32.astype(np.float16).view(np.uint16)
    if xd == BF16:
        u = x32.view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return x32


def bench_qmm(ctx, hip, M, K, N, bits, gs, xd, sbd, od, steps, warmup, kernel, copies=COPIES, seed=1,
              keep=False, outliers=False):
    """Times `steps` launches over `copies` rotating weight sets; keep=True
    also returns copy 0's inputs and output (downloaded) for the parity check.
    r["digest_match"]: copy 0's weights against the committed digests."""
    from mlx_amd import runtime
    xh = x_host(M, K, xd, seed)
    xb = ctx.upload(xh)
    sets = make_weights(ctx, N, K, bits, gs, sbd, copies, seed, outliers)
    sbnp = runtime.np_dtype(sbd)
    wq0, s0, b0 = sets[0]
    wq0h = wq0.download(np.uint32, (N, K * bits // 32))
    s0h, b0h = s0.download(sbnp, (N, K // gs)), b0.download(sbnp, (N, K // gs))
    dm = digest_match(K, N, bits, gs, sbd, seed, outliers, wq0h, s0h, b0h)
    out = ctx.alloc(M * N * runtime.esize(od))
    stream = ctx.stream

    def step(i):
        wq, s, b = sets[i % copies]
        ctx.quantized_matmul(xb, wq, s, b, out, M, K, N, gs, bits, xd, sbd, od, kernel)

    # the timed launches: the same op through the same table entry, called
    # from a C loop (a Python call per launch costs ~6 us of host time, about
    # as long as the M = 1 kernel runs, so a slow host would leave the GPU
    # idle between launches)
    L = ceiling_lib()
    fn = ctypes.cast(ctx.q.op_quantized_matmul_ex, ctypes.c_void_p)
    handles = [(ctypes.c_void_p * copies)(*[st[j].handle for st in sets]) for j in range(3)]

    def loop(first, n):
        rc = L.lux_bench_qmm_loop(fn, ctx.handle, xb.handle, handles[0], handles[1], handles[2], copies,
                                  out.handle, M, K, N, gs, bits, xd, sbd, od, kernel, first, n)
        if rc != 0:
            raise RuntimeError(f"op_quantized_matmul_ex failed in the C loop: {rc}")

    r = time_launches(hip, stream, step, steps, max(warmup, copies), loop)
    r["graph_ms_per_launch"] = time_graph(hip, stream, step)
    r["steps"] = steps
    r["digest_match"] = dm
    if keep:
        step(0)
        ctx.sync()
        r["y"] = out.download(runtime.np_dtype(od), (M, N))
        r["x"] = xh
        r["w_q"], r["s"], r["b"] = wq0h, s0h, b0h
    for t in [xb, out] + [b for st in sets for b in st]:
        t.free()
    return r


# ---- ceiling leg -----------------------------------------------------------

def ceiling_lib():
    path = os.path.join(ROOT, "mlx_amd", "lib", "libluxgpu_ceiling.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run python -c 'import __graft_entry__ as g; g.build()'")
    L = ctypes.CDLL(path)
    L.lux_ceiling_empty.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    L.lux_ceiling_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    L.lux_ceiling_empty_loop.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.POINTER(ctypes.c_float)]
    L.lux_ceiling_read_loop.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint64,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    L.lux_bench_qmm_loop.argtypes = [ctypes.c_void_p] * 3 + [ctypes.POINTER(ctypes.c_void_p)] * 3 + \
        [ctypes.c_int, ctypes.c_void_p] + [ctypes.c_int] * 11
    L.lux_bench_rng_normal_f32.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float,
                                           ctypes.c_float]
    L.lux_bench_rng_u32.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64]
    return L


def ceiling_leg(ctx, hip, nbytes, steps, warmup, blocks):
    """Empty kernel (`blocks` blocks) and a plain read of nbytes over COPIES
    rotating buffers, timed as the GEMV is."""
    L = ceiling_lib()
    stream = ctx.stream
    stride = (nbytes + (2 << 20) - 1) // (2 << 20) * (2 << 20)
    buf = hip.malloc(stride * COPIES)
    sink = hip.malloc(1 << 20)
    hip.memset(buf, 0x3C, stride * COPIES)
    base = buf.value
    out = {}
    try:
        def read(i):
            hip.ck(L.lux_ceiling_read(ctypes.c_void_p(base + (i % COPIES) * stride), nbytes, sink,
                                      ctypes.c_void_p(stream)), "lux_ceiling_read")

        def empty(i):
            hip.ck(L.lux_ceiling_empty(blocks, sink, ctypes.c_void_p(stream)), "lux_ceiling_empty")

        def read_loop(first, n):
            # timed like the quantized matmul: the launches issued from C
            hip.ck(L.lux_ceiling_read_loop(ctypes.c_void_p(base), stride, COPIES, nbytes, sink,
                                           ctypes.c_void_p(stream), first, n), "lux_ceiling_read_loop")

        for name, fn, loop in (("empty", empty, None), ("read", read, read_loop)):
            r = time_launches(hip, stream, fn, steps, warmup, loop)
            g = time_graph(hip, stream, fn)
            us = r["event_ms_per_launch"] * 1e3
            out[name] = {"us_per_launch": round(us, 3), "graph_us_per_launch": round(g * 1e3, 3)}
            if name == "read":
                out[name]["frac_of_peak"] = round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                out[name]["graph_frac_of_peak"] = round(nbytes / g / 1e6 / HBM_PEAK_GBS, 4)
        # the same empty launches issued from a C loop (no Python call per
        # launch), after the leg's own warm-up
        ms = ctypes.c_float()
        hip.ck(L.lux_ceiling_empty_loop(steps, blocks, sink, ctypes.c_void_p(stream), ctypes.byref(ms)),
               "lux_ceiling_empty_loop")
        out["empty"]["c_loop_us_per_launch"] = round(ms.value * 1e3 / steps, 3)
        out["bytes"] = nbytes
        out["empty_blocks"] = blocks
    finally:
        hip.sync(stream)
        hip.free(buf)
        hip.free(sink)
    return out


# ---- CPU baseline and parity (the oracle as checker) ----------------------

def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"nproc": usable, "cpu_count": os.cpu_count(), "model": model,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def _timed(fn, budget_s, min_calls=10, warmups=3):
    """`warmups` untimed calls, then timed calls until there are at least
    min_calls and budget_s seconds of them; the per-call seconds."""
    for _ in range(warmups):
        fn()
    ts, t_start = [], time.perf_counter()
    while len(ts) < min_calls or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return ts


def ref_cpu_backend():
    """The reference CPU backend built from its source (oracle/_ref), or None."""
    path = os.path.join(ROOT, "oracle", "_ref", "libref_cpu_backend.so")
    if not os.path.exists(path):
        return None
    from mlx_amd import abi
    lib = ctypes.CDLL(path)
    desc = abi.BackendDesc()
    if not abi.INIT_FN(("cpu_backend_init", lib))(ctypes.byref(desc)):
        return None
    return lib, desc


def cpu_baseline(M, K, N, bits, gs, budget_s=4.0):
    """The oracle's OpenMP GEMV (a port of the path: the reference has no
    quantized op) on all of this process's cores and on one core, plus the
    reference's own composition: host dequantize (the oracle) to f32 W^T
    [K, N], then the reference CPU backend's op_matmul_f32 (naive, OpenMP)."""
    from oracle import oracle as O
    info = host_info()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or info["nproc"] or 1
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, F16, F16, seed=1)
    wb = weight_bytes(N, K, bits, gs, F16)

    def port(t):
        return lambda: O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F16, F16, F16, variant="omp", threads=t)

    t_all = _timed(port(threads), budget_s)
    t_one = _timed(port(1), budget_s)
    med_all, med_one = float(np.median(t_all)), float(np.median(t_one))
    out = {"value": round(wb / med_all / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"median of {len(t_all)} timed calls (after 3 warm-up calls) of the OpenMP CPU "
                     f"quantized GEMV (oracle), M={M} K={K} N={N} {bits}-bit g{gs} f16, "
                     f"{sum(t_all):.1f} s on {threads} threads",
           "mean_value": round(wb * len(t_all) / sum(t_all) / 1e9, 3),
           "one_core": {"value": round(wb / med_one / 1e9, 3), "unit": "GB/s", "cores": 1,
                        "sample": f"median of {len(t_one)} calls after 3 warm-ups, {sum(t_one):.1f} s"},
           "host": info}
    ref = ref_cpu_backend()
    if ref is None:
        out["reference_composition"] = None
    else:
        _, desc = ref
        vt = desc.vtbl.contents
        ctx = vt.create_context(0)
        xf = np.ascontiguousarray(O.to_f32(x, F16))
        bx = vt.buffer_alloc_with_data(ctx, xf.ctypes.data, xf.nbytes)
        bw = vt.buffer_alloc(ctx, K * N * 4)
        by = vt.buffer_alloc(ctx, M * N * 4)

        def compose():
            wt = np.ascontiguousarray(O.dequantize(w_q, s, b, K, gs, bits, F16).T)
            if vt.buffer_copy_from_host(ctx, bw, wt.ctypes.data, wt.nbytes) != 0:
                raise RuntimeError("reference buffer_copy_from_host")
            if vt.op_matmul_f32(ctx, bx, bw, by, M, K, N) != 0:
                raise RuntimeError("reference op_matmul_f32")

        t_ref = _timed(compose, 0.0)
        for h in (bx, bw, by):
            vt.buffer_free(ctx, h)
        vt.destroy_context(ctx)
        out["reference_composition"] = {
            "value": round(wb / float(np.median(t_ref)) / 1e9, 3), "unit": "GB/s", "kind": "reference",
            "cores": int(os.environ.get("OMP_NUM_THREADS", "0")) or info["nproc"],
            "sample": f"median of {len(t_ref)} calls (after 3 warm-ups) of host dequantize to f32 W^T + "
                      f"reference cpu_op_matmul_f32 (src/cpu_backend.cpp:243-266, OpenMP), {sum(t_ref):.1f} s"}
    return out


def rel_err(y, want, od):
    from oracle import oracle as O
    yf = O.to_f32(y, od).astype(np.float64) if od != F32 else y.astype(np.float64)
    wf = O.to_f32(want, od).astype(np.float64) if od != F32 else want.astype(np.float64)
    return float(np.abs(yf - wf).max() / max(np.abs(wf).max(), 1e-30))


def parity(cases, threads):
    """max|d|/max|y| of each GPU output against the oracle (the oracle's
    OpenMP form, fp32 accumulation) on the same inputs; GEMM outputs also
    against the exact-weight form."""
    from oracle import oracle as O
    res = {}
    for name, c in cases.items():
        M, K, N, gs, bits, xd, sbd, od, gemm = c["shape"]
        r = c["run"]
        args = (r["x"], r["w_q"], r["s"], r["b"], M, K, N, gs, bits, xd, sbd)
        want = O.quantized_matmul(*args, od, variant="omp", threads=threads, w_round=xd if gemm else F32)
        e = {"max_rel": rel_err(r["y"], want, od), "out_dtype": {F16: "f16", BF16: "bf16", F32: "f32"}[od]}
        if gemm:
            exact = O.quantized_matmul(*args, od, variant="omp", threads=threads)
            e["max_rel_vs_exact_weights"] = rel_err(r["y"], exact, od)
        res[name] = e
    return res


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


def parse_shape(spec):
    """'M,K,N,bits,group,x' (x: f16, bf16 or f32; scales and output in the
    same type) -> a SWEEP-style tuple named 'shape'."""
    f = spec.split(",")
    if len(f) != 6:
        raise SystemExit(f"--shape wants M,K,N,bits,group,x; got {spec!r}")
    dt = {"f16": F16, "bf16": BF16, "f32": F32}[f[5]]
    return ("shape", int(f[0]), int(f[1]), int(f[2]), int(f[3]), int(f[4]), dt, dt, dt)


def copies_for(wb):
    """Rotated weight copies: together at least 2.2 x the 256 MB Infinity
    Cache, so each launch streams its weights from HBM (4..64 copies)."""
    return max(4, min(64, -(-int(2.2 * (256 << 20)) // wb)))


# the BASELINE configs the headline line does not already time (configs[0],
# [2] and [4]; [1] and [3] are the headline, decode and GEMM legs)
CONFIG_LEGS = [s for s in SWEEP if s[0] in ("c0", "c2", "c4")]


def config_legs(ctx, hip, steps, warmup, keep=False):
    """One entry per CONFIG_LEGS shape, timed as the headline is: the kernel
    class AUTO picks, mean and median us per launch, graph replays, and the
    weight-byte and flop rates with their roofline fractions.  keep=True
    also returns the c2 run (inputs and output) for the parity check."""
    from mlx_amd import abi
    out, runs = {}, {}
    for name, M, K, N, bits, gs, xd, sbd, od in CONFIG_LEGS:
        wb = weight_bytes(N, K, bits, gs, sbd)
        r = bench_qmm(ctx, hip, M, K, N, bits, gs, xd, sbd, od, steps, warmup, abi.KERNEL_AUTO,
                      copies=copies_for(wb), keep=keep and name == "c2", outliers=name == "c4")
        t = r["event_ms_per_launch"] * 1e-3
        flops = 2.0 * M * N * K
        key = f"{name}_m{M}_{bits}bit"
        out[key] = {"M": M, "K": K, "N": N, "bits": bits, "group_size": gs,
                    "kernel": ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od),
                    "kernel_us_avg": round(t * 1e6, 3), "kernel_us_median": r["per_launch_us"]["median"],
                    "graph_us": round(r["graph_ms_per_launch"] * 1e3, 3),
                    "weight_GBs": round(wb / t / 1e9, 1), "hbm_frac": round(wb / t / 1e9 / HBM_PEAK_GBS, 4),
                    "tflops": round(flops / t / 1e12, 2),
                    "mfma_frac": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4),
                    "copies": copies_for(wb), "digest_match": r["digest_match"]}
        if keep and name == "c2":
            runs["c2"] = r
    return out, runs


def sweep(ctx, hip, steps, only=None, table=SWEEP):
    """One line per config: kernel AUTO picks, per-launch time (stream and
    graph replays), weight GB/s and TFLOP/s with their roofline fractions."""
    from mlx_amd import abi
    for name, M, K, N, bits, gs, xd, sbd, od in table:
        if only and name not in only:
            continue
        copies = 4 if M >= 256 else copies_for(weight_bytes(N, K, bits, gs, sbd))
        r = bench_qmm(ctx, hip, M, K, N, bits, gs, xd, sbd, od, steps, 8, abi.KERNEL_AUTO, copies=copies,
                      outliers=name == "c4")
        t = r["event_ms_per_launch"] * 1e-3
        wb = weight_bytes(N, K, bits, gs, sbd)
        flops = 2.0 * M * N * K
        print(json.dumps({"config": name, "M": M, "K": K, "N": N, "bits": bits, "group_size": gs,
                          "kernel": ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od), "us": round(t * 1e6, 3),
                          "us_median": r["per_launch_us"]["median"],
                          "graph_us": round(r["graph_ms_per_launch"] * 1e3, 3),
                          "weight_GBs": round(wb / t / 1e9, 1), "hbm_frac": round(wb / t / 1e9 / HBM_PEAK_GBS, 4),
                          "tflops": round(flops / t / 1e12, 2),
                          "mfma_frac": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4),
                          "digest_match": r["digest_match"]}), flush=True)


def decode_legs(ctx, hip, K, N, bits, gs, steps, warmup):
    """configs[1] at M=4 and M=8: same weight bytes as M=1, 4x / 8x the math."""
    from mlx_amd import abi
    out = {}
    wb = weight_bytes(N, K, bits, gs, F16)
    for m in (4, 8):
        r = bench_qmm(ctx, hip, m, K, N, bits, gs, F16, F16, F16, steps, warmup, abi.KERNEL_AUTO)
        t = r["event_ms_per_launch"] * 1e-3
        out[f"M{m}"] = {"kernel": ctx.kernel_name(m, K, N, gs, bits, F16, F16, F16),
                        "kernel_us_avg": round(t * 1e6, 3), "kernel_us_median": r["per_launch_us"]["median"],
                        "graph_us": round(r["graph_ms_per_launch"] * 1e3, 3),
                        "weight_GBs": round(wb / t / 1e9, 1), "hbm_frac": round(wb / t / 1e9 / HBM_PEAK_GBS, 4),
                        "digest_match": r["digest_match"]}
    return out


GEMV_PROFILE = os.path.join(ROOT, "profiles", "qgemv_line_m1_k4096_n14336_4bit_g64_f16.md")


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and parity leg")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true")
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the headline line, one JSON line per BASELINE config")
    ap.add_argument("--only", default="", help="with --sweep: comma-separated config names (c0..c4)")
    ap.add_argument("--shape", action="append", default=[], metavar="M,K,N,BITS,GROUP,X",
                    help="instead of the headline line, a sweep line for this shape (repeatable; for profiling)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the configs[1] M=4 and M=8 decode legs (for profiling)")
    ap.add_argument("--ceiling-only", action="store_true", help="only the ceiling leg (for profiling)")
    ap.add_argument("--gemm-only", action="store_true", help="only the configs[3] GEMM legs (for profiling)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a device-to-device copy of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy(Hip(), args.calibrate_copy)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the plugin path is single-device; DESIGN.md section 7 gives how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    from mlx_amd import abi, runtime
    hip = Hip()
    ctx = runtime.Context(0)
    M, K, N, bits, gs = 1, 4096, 14336, 4, 64
    wb = weight_bytes(N, K, bits, gs, F16)
    if args.sweep:
        sweep(ctx, hip, min(args.steps, 256), [s for s in args.only.split(",") if s])
        ctx.close()
        return
    if args.shape:
        sweep(ctx, hip, min(args.steps, 256), None, [parse_shape(s) for s in args.shape])
        ctx.close()
        return
    if args.decode_only:
        print(json.dumps({"decode_m4_m8": decode_legs(ctx, hip, K, N, bits, gs, args.steps, args.warmup)}),
              flush=True)
        ctx.close()
        return
    if args.ceiling_only:
        print(json.dumps({"ceiling": ceiling_leg(ctx, hip, wb, args.steps, args.warmup, 512)}), flush=True)
        ctx.close()
        return

    def gemm_legs(keep):
        gemm, runs = {}, {}
        for n in (4096, 14336):
            if ctx.select_kernel(2048, 4096, n, 64, 4, BF16) != abi.KERNEL_GEMM:
                break
            steps = min(args.steps, 256)
            rg = bench_qmm(ctx, hip, 2048, 4096, n, 4, 64, BF16, BF16, BF16, steps, args.warmup,
                           abi.KERNEL_AUTO, copies=4, keep=keep and n == 4096)
            flops = 2.0 * 2048 * 4096 * n
            tf = flops / (rg["event_ms_per_launch"] * 1e-3) / 1e12
            gemm[f"N{n}"] = {"kernel": ctx.kernel_name(2048, 4096, n, 64, 4, BF16, BF16, BF16),
                             "tflops": round(tf, 2), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                             "kernel_us_avg": round(rg["event_ms_per_launch"] * 1e3, 2),
                             "kernel_us_median": rg["per_launch_us"]["median"],
                             "per_launch_us": rg["per_launch_us"],
                             "graph_us": round(rg["graph_ms_per_launch"] * 1e3, 2),
                             "wall_tflops": round(flops * rg["steps"] / rg["wall_s"] / 1e12, 2),
                             "digest_match": rg["digest_match"]}
            runs[n] = rg
        return gemm, runs

    if args.gemm_only:
        print(json.dumps({"gemm_m2048": gemm_legs(False)[0]}), flush=True)
        ctx.close()
        return

    keep = not args.no_cpu
    r = bench_qmm(ctx, hip, M, K, N, bits, gs, F16, F16, F16, args.steps, args.warmup, abi.KERNEL_AUTO, keep=keep)
    value = wb * r["steps"] / r["wall_s"] / 1e9
    t = r["event_ms_per_launch"] * 1e-3
    achieved = wb / t / 1e9
    line = {
        "metric": "weight GB/s (%HBM peak) at M=1 & TFLOP/s (%MFMA peak) at M=2048, 4-bit",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] * 1e3 / r["steps"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "runtime_env": {"HIP_FORCE_DEV_KERNARG": os.environ.get("HIP_FORCE_DEV_KERNARG")},
        "data": "synthetic, seed 1, from the test fixtures' portable generator (xoshiro256** + Box-Muller): "
                "x~N(0,1) f16, W~N(0,0.02) quantized on the GPU (4-bit, group 64, f16 scales/biases); "
                "16 rotated weight copies; copy 0 hashes to the committed digests: " + str(r["digest_match"]),
        "config": {"workload": "configs[1] decode GEMV M=1", "M": M, "K": K, "N": N, "bits": bits,
                   "group_size": gs, "kernel": ctx.kernel_name(M, K, N, gs, bits, F16, F16, F16),
                   "hbm_pct": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(GEMV_PROFILE),
                     "kernel": ctx.kernel_name(M, K, N, gs, bits, F16, F16, F16), "kernel_us_avg": round(t * 1e6, 3),
                     "kernel_us_median": r["per_launch_us"]["median"], "per_launch_us": r["per_launch_us"],
                     "graph_us_per_launch": round(r["graph_ms_per_launch"] * 1e3, 3),
                     "graph_frac": round(wb / r["graph_ms_per_launch"] / 1e6 / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": wb,
                     "timing": "HIP events around the timed launches on the plugin stream, issued from a C loop "
                               "through the plugin's op table"},
    }
    if not args.no_ceiling:
        line["ceiling"] = ceiling_leg(ctx, hip, wb, args.steps, args.warmup, 512)
    line["decode_m4_m8"] = decode_legs(ctx, hip, K, N, bits, gs, min(args.steps, 1024), args.warmup)
    gemm_runs = {}
    if not args.no_gemm:
        line["gemm_m2048"], gemm_runs = gemm_legs(keep)
    line["configs"], cfg_runs = config_legs(ctx, hip, min(args.steps, 256), args.warmup, keep)
    # c2's kernel family decides its semantics (the GEMM kernels dequantize
    # to the activation type before the multiply)
    c2_gemm = ctx.select_kernel(32, 8192, 8192, 128, 8, BF16) == abi.KERNEL_GEMM
    if keep:
        c2 = cfg_runs["c2"]
        c2f = bench_qmm(ctx, hip, 32, 8192, 8192, 8, 128, BF16, BF16, F32, 16, 4, abi.KERNEL_AUTO,
                        copies=4, keep=True)
    ctx.close()
    if keep:
        cb = cpu_baseline(M, K, N, bits, gs)
        cases = {"c1_m1_f16": {"shape": (M, K, N, gs, bits, F16, F16, F16, False), "run": r},
                 "c2_bf16": {"shape": (32, 8192, 8192, 128, 8, BF16, BF16, BF16, c2_gemm), "run": c2},
                 "c2_f32out": {"shape": (32, 8192, 8192, 128, 8, BF16, BF16, F32, c2_gemm), "run": c2f}}
        if 4096 in gemm_runs:
            cases["c3_n4096_bf16"] = {"shape": (2048, 4096, 4096, 64, 4, BF16, BF16, BF16, True),
                                      "run": gemm_runs[4096]}
        cb["parity"] = parity(cases, cb["cores"])
        line["cpu_baseline"] = cb
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
