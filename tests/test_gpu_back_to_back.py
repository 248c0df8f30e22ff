"""Launches issued back to back on the context stream with no host
synchronization between them -- the pattern the benchmark times.

The GEMMs that split work across blocks keep tile counters and flags in the
context's workspace: the split last round of both large GEMMs (halves meet
by the launch's epoch; counters never reset), the register-W GEMM's K parts
and the split-K small-M GEMM (counters the last block returns to zero).
Each case here uploads its inputs once, enqueues LAUNCHES launches into
separate output buffers without a synchronize, synchronizes once, then
checks launch 0 against the oracle and every later launch bit for bit
against launch 0: a counter or flag one launch left behind would change a
later launch's sums (or leave a tile NaN).  The pattern follows the
backend-agnostic checks of the reference's own tests
(test/test_core.cpp:95-117: run whatever backend is loaded, compare against
known values).
"""
import numpy as np
import pytest

from qmm_util import BF16, F16, F32, check_output

pytestmark = pytest.mark.gpu

LAUNCHES = 8

# name, (M, K, N, bits, group, x dtype, scale dtype, out dtype, kernel), GEMM
# semantics, the kernel that runs
CASES = [
    # configs[3] N = 14336: 896 tiles, the last 128 as two K halves each
    ("c3_n14336_split_last_round", (2048, 4096, 14336, 4, 64, BF16, BF16, BF16, 0), True, "qgemm_rw_kernel"),
    # 128 tiles of 128 x 256, each in two K parts
    ("rw_k_parts", (1024, 4096, 4096, 4, 64, BF16, BF16, F32, 2), True, "qgemm_rw_kernel"),
    # 3-bit codes: the LDS-dequant GEMM, 128 tiles of 256 x 128, every one
    # as two K halves
    ("gemm_all_tiles_split", (1024, 4096, 4096, 3, 64, BF16, BF16, F32, 2), True, "qgemm_kernel"),
    # split-K small-M GEMM: K % 1024 != 0, K parts meet in the workspace
    ("small_m_split_k", (64, 3584, 4096, 3, 64, F16, F16, F16, 0), True, "qgemm_sk_kernel"),
    # split-K small-M GEMM, 4-bit, ragged N
    ("small_m_split_k_4bit", (40, 3200, 6000, 4, 64, F16, F16, F32, 0), True, "qgemm_sk_kernel"),
]


@pytest.mark.parametrize("name,shape,gemm,kernel", CASES, ids=[c[0] for c in CASES])
def test_back_to_back_launches(ctx, oracle, name, shape, gemm, kernel):
    from mlx_amd import runtime
    O = oracle
    M, K, N, bits, gs, xd, sbd, od, kern = shape
    print(f"[case] back to back {name}: M={M} K={K} N={N} bits={bits} g={gs} kernel={kern}", flush=True)
    assert ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od, kern) == kernel, "case meant for " + kernel
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=8100 + N + M)
    ins = [ctx.upload(a) for a in (x, w_q, s, b)]
    outs = [ctx.alloc(M * N * runtime.esize(od)) for _ in range(LAUNCHES)]
    try:
        for o in outs:
            ctx.quantized_matmul(*ins, o, M, K, N, gs, bits, xd, sbd, od, kern)
        ctx.sync()
        ys = [o.download(runtime.np_dtype(od), (M, N)) for o in outs]
    finally:
        for buf in ins + outs:
            buf.free()
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="omp",
                              w_round=xd if gemm else F32)
    check_output(O, ys[0], want, od, f"{name} launch 0")
    for i in range(1, LAUNCHES):
        assert np.array_equal(ys[i].view(np.uint8), ys[0].view(np.uint8)), f"{name}: launch {i} differs from launch 0"
