"""The allocation-free entry point lux_gpu_quantized_matmul_noalloc, called
through the C ABI on raw device pointers and a caller stream, against the
context op op_quantized_matmul_ex on the same inputs: bit for bit (the same
kernels, and the same K split, since its static scratch is the size of a
context's workspace), and within the output gate of the oracle.  Two calls
in a row share the scratch, the second with a smaller input; the first two
run the split-K GEMM with its parts meeting in the scratch, the next two the
large GEMM with the two K halves of its tiles meeting there, so a counter or
flag left nonzero by one call would break the next; the fifth runs the large
GEMM on one block per CU (more tiles than CUs, 16-bit output), its blocks
going on from a whole tile to a K half.
"""
import ctypes
import os

import numpy as np
import pytest

from qmm_util import BF16, F16, F32, check_output

pytestmark = pytest.mark.gpu

# (M, K, N, bits, group size, x dtype, scales dtype, out dtype, kernel)
CALLS = [
    (64, 3584, 4096, 3, 64, F16, F16, F16, 0),     # split-K GEMM, 7 K parts, 224 blocks
    (17, 1152, 200, 4, 32, BF16, BF16, F32, 2),    # split-K GEMM, 3 K parts, 6 blocks
    (512, 1024, 1024, 4, 64, BF16, BF16, F32, 2),  # large GEMM, 16 tiles, each in two K halves
    (300, 512, 200, 4, 64, F16, F16, F16, 2),      # large GEMM, 4 ragged tiles, each in two K halves
    (2000, 1024, 4360, 4, 64, BF16, BF16, BF16, 2),  # large GEMM, one block per CU: 288 ragged tiles, 32 in K halves
    (1, 4096, 512, 4, 64, F16, F16, F16, 0),       # a GEMV: no scratch
]


class _Hip:
    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so", mode=os.RTLD_NOW | os.RTLD_GLOBAL)

    def ck(self, rc, what):
        assert rc == 0, f"{what}: hipError {rc}"

    def upload(self, a):
        p = ctypes.c_void_p()
        self.ck(self.L.hipMalloc(ctypes.byref(p), ctypes.c_size_t(max(1, a.nbytes))), "hipMalloc")
        self.ck(self.L.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1), "hipMemcpy")
        return p

    def alloc(self, n):
        p = ctypes.c_void_p()
        self.ck(self.L.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)), "hipMalloc")
        self.ck(self.L.hipMemset(p, 0xFF, ctypes.c_size_t(n)), "hipMemset")
        return p

    def download(self, p, dtype, shape):
        a = np.empty(shape, dtype)
        self.ck(self.L.hipMemcpy(a.ctypes.data_as(ctypes.c_void_p), p, ctypes.c_size_t(a.nbytes), 2), "hipMemcpy")
        return a

    def free(self, p):
        self.ck(self.L.hipFree(p), "hipFree")


def _entry():
    import mlx_amd
    lib = ctypes.CDLL(mlx_amd.PLUGIN_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    f = lib.lux_gpu_quantized_matmul_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8 + [ctypes.c_int, ctypes.c_void_p]
    return f


def test_noalloc_matches_context_op(ctx, oracle):
    from mlx_amd import runtime
    O = oracle
    f = _entry()
    hip = _Hip()
    stream = ctypes.c_void_p()
    hip.ck(hip.L.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    try:
        for i, (M, K, N, bits, gs, xd, sbd, od, kern) in enumerate(CALLS):
            print(f"[case] noalloc call {i}: M={M} K={K} N={N} b={bits} g={gs} x={xd} kernel={kern}", flush=True)
            x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=700 + i)
            ptrs = [hip.upload(np.ascontiguousarray(a)) for a in (x, w_q, s, b)]
            nbytes = M * N * runtime.esize(od)
            out = hip.alloc(nbytes)
            try:
                rc = f(*ptrs, out, M, K, N, gs, bits, xd, sbd, od, kern, stream)
                assert rc == 0, f"noalloc returned {rc}"
                hip.ck(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
                got = hip.download(out, runtime.np_dtype(od), (M, N))
            finally:
                for p in ptrs + [out]:
                    hip.free(p)
            want = runtime.run_quantized_matmul(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, kern)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"call {i} differs from the context op"
            gemm = ctx.select_kernel(M, K, N, gs, bits, xd, sbd) == 2 if kern == 0 else kern == 2
            ref = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="omp",
                                     w_round=xd if gemm else F32)
            check_output(O, got, ref, od, f"noalloc call {i}")
    finally:
        hip.ck(hip.L.hipStreamDestroy(stream), "hipStreamDestroy")


def test_noalloc_back_to_back(ctx, oracle):
    """The split-K, split-last-round and persistent calls of CALLS enqueued
    on one stream with no synchronize between them (the scratch's counters
    and flags must be back at zero when the next call starts), then each
    output against the context op on the same inputs, bit for bit."""
    from mlx_amd import runtime
    O = oracle
    f = _entry()
    hip = _Hip()
    stream = ctypes.c_void_p()
    hip.ck(hip.L.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    calls, held = CALLS[:5] * 2, []
    try:
        for i, (M, K, N, bits, gs, xd, sbd, od, kern) in enumerate(calls):
            print(f"[case] noalloc back-to-back call {i}: M={M} K={K} N={N} b={bits} kernel={kern}", flush=True)
            x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=700 + i % 5)
            ptrs = [hip.upload(np.ascontiguousarray(a)) for a in (x, w_q, s, b)]
            out = hip.alloc(M * N * runtime.esize(od))
            held.append((ptrs, out, (x, w_q, s, b), (M, K, N, bits, gs, xd, sbd, od, kern)))
            rc = f(*ptrs, out, M, K, N, gs, bits, xd, sbd, od, kern, stream)
            assert rc == 0, f"noalloc returned {rc}"
        hip.ck(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
        for i, (ptrs, out, host, (M, K, N, bits, gs, xd, sbd, od, kern)) in enumerate(held):
            got = hip.download(out, runtime.np_dtype(od), (M, N))
            want = runtime.run_quantized_matmul(ctx, *host, M, K, N, gs, bits, xd, sbd, od, kern)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"call {i} differs from the context op"
    finally:
        for ptrs, out, _, _ in held:
            for p in ptrs + [out]:
                hip.free(p)
        hip.ck(hip.L.hipStreamDestroy(stream), "hipStreamDestroy")


def test_noalloc_graph_capture(ctx, oracle):
    """One split-K call (parts meeting in the scratch) captured into a HIP
    graph after an eager call on the device, the graph replayed three times
    with the host's own synchronizations and downloads between replays;
    every replay equals the context op bit for bit."""
    from mlx_amd import runtime
    O = oracle
    f = _entry()
    hip = _Hip()
    M, K, N, bits, gs, xd, sbd, od, kern = CALLS[0]
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=760)
    want = runtime.run_quantized_matmul(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, kern)
    stream = ctypes.c_void_p()
    hip.ck(hip.L.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    ptrs = [hip.upload(np.ascontiguousarray(a)) for a in (x, w_q, s, b)]
    out = hip.alloc(M * N * runtime.esize(od))
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        # the eager call sets the scratch up on this device (a first call may not be captured)
        assert f(*ptrs, out, M, K, N, gs, bits, xd, sbd, od, kern, stream) == 0
        hip.ck(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
        hip.ck(hip.L.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")  # global mode
        rc = f(*ptrs, out, M, K, N, gs, bits, xd, sbd, od, kern, stream)
        hip.ck(hip.L.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
        assert rc == 0, f"captured noalloc call returned {rc}"
        hip.ck(hip.L.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
        for rep in range(3):
            print(f"[case] noalloc graph replay {rep}", flush=True)
            hip.ck(hip.L.hipMemset(out, 0xFF, ctypes.c_size_t(M * N * runtime.esize(od))), "hipMemset")
            hip.ck(hip.L.hipGraphLaunch(exe, stream), "hipGraphLaunch")
            hip.ck(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
            got = hip.download(out, runtime.np_dtype(od), (M, N))
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"replay {rep} differs"
    finally:
        if exe.value:
            hip.L.hipGraphExecDestroy(exe)
        if graph.value:
            hip.L.hipGraphDestroy(graph)
        for p in ptrs + [out]:
            hip.free(p)
        hip.ck(hip.L.hipStreamDestroy(stream), "hipStreamDestroy")


def test_noalloc_errors():
    """Errors come back before any device work: null pointers, a bad shape.
    The pointers are real (small) device allocations, so a check that ran
    after a launch would still not touch unmapped memory."""
    f = _entry()
    hip = _Hip()
    p = hip.alloc(4096)
    try:
        assert f(None, p, p, p, p, 16, 256, 8, 64, 4, F16, F16, F16, 0, None) == 1  # INVALID_ARGUMENT
        assert f(p, p, p, p, p, 16, 100, 8, 64, 4, F16, F16, F16, 0, None) == 1     # K % group size
        assert f(p, p, p, p, p, 16, 256, 8, 64, 7, F16, F16, F16, 0, None) != 0     # bits outside the format
        assert f(p, p, p, p, p, 16, 256, 8, 64, 4, F16, F16, F16, 9, None) == 1     # unknown kernel
    finally:
        hip.free(p)
