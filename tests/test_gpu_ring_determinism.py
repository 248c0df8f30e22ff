"""Repeat-launch determinism over the layouts of the kernels whose waits or
cross-block meetings depend on them.

The small-M GEMM (qgemm_small) and the mid-M GEMV (qgemv_mid) stage x, W and
the scales in per-wave LDS rings filled by buffer->LDS transfers, and every
step waits on a compile-time count of the transfers issued after the x it
reads.  A count that is too large for some layout (code width, scale dtype,
group size, one or two 32-row M tiles, one or two column tiles per block:
each changes the ring's slots and the transfers per issue) lets a step read
a slot before its data landed: the output then changes from launch to
launch.  One such count was found this way (the first step of the 8-bit,
f32-scale, group-32 two-tile blocks); the oracle comparisons elsewhere ran
those shapes once and passed.

Each case runs LAUNCHES launches back to back into separate output buffers
(fp32, so that every bit of the sums shows, but for the register-W GEMM's
persistent grid, which stores 16-bit outputs), synchronizes once and checks
that all of them equal the first bit for bit.  K = 1024 gives each wave one
super-step, so the prologue's issues and the first steps' waits are most of
the kernel.  The inputs are random codes with finite scales, biases and x:
the oracle checks of these kernels are in test_gpu_parity.py.

The GEMMs get the same check over scale dtype x group size (which set the
register-W GEMM's scale windows, unroll and compile-time wait counts): the
register-W GEMM with K parts meeting in the workspace and on its persistent
grid with a split last round, the split-K small-M GEMM (K parts, counters
the last part returns to zero) and the LDS-dequant GEMM for the other code
widths.  So do the GEMV kernels AUTO picks for M = 1..8.
"""
import numpy as np
import pytest

from qmm_util import BF16, F16, F32

pytestmark = pytest.mark.gpu

LAUNCHES = 32
BITS = [2, 3, 4, 5, 6, 8]
SB = [F16, BF16, F32]
GROUPS = [32, 64, 128]


def _values(rng, n, lo, hi, dtype):
    v = rng.uniform(lo, hi, n).astype(np.float32)
    if dtype == F32:
        return v
    if dtype == F16:
        return v.astype(np.float16)
    return (v.view(np.uint32) >> 16).astype(np.uint16)  # bf16 bits (truncated)


def _repeat(ctx, M, K, N, gs, bits, xd, sbd, kernel, name, seed, od=F32, launches=LAUNCHES):
    """kernel: the kernel the case is meant for, or None for whatever AUTO
    picks."""
    from mlx_amd import abi, runtime
    if kernel is None:
        kern = abi.KERNEL_AUTO
        name += " (" + str(ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od, kern)) + ")"
    else:
        kern = abi.KERNEL_GEMV if kernel.startswith("qgemv") else abi.KERNEL_GEMM
        assert ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od, kern) == kernel, "case meant for " + kernel
    rng = np.random.default_rng(seed)
    x = _values(rng, M * K, -1.0, 1.0, xd)
    w_q = rng.integers(0, 2**32, N * K * bits // 32, dtype=np.uint32)
    s = _values(rng, N * (K // gs), 0.004, 0.02, sbd)
    b = _values(rng, N * (K // gs), -0.2, -0.05, sbd)
    ins = [ctx.upload(a) for a in (x, w_q, s, b)]
    outs = [ctx.alloc(M * N * runtime.esize(od)) for _ in range(launches)]
    try:
        print(f"[case] {name}", flush=True)
        for o in outs:
            ctx.quantized_matmul(*ins, o, M, K, N, gs, bits, xd, sbd, od, kern)
        ctx.sync()
        ys = [o.download(runtime.np_dtype(od), (M, N)) for o in outs]
    finally:
        for t in ins + outs:
            t.free()
    assert np.isfinite(ys[0].astype(np.float32) if od != BF16 else
                       (ys[0].astype(np.uint32) << 16).view(np.float32)).all(), f"{name}: non-finite output"
    bad = [i for i, y in enumerate(ys) if not np.array_equal(y, ys[0])]
    assert not bad, f"{name}: launches {bad} differ from launch 0"


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sbd", SB, ids=["sb_f16", "sb_bf16", "sb_f32"])
def test_small_gemm_rings_repeat(ctx, bits, sbd):
    """qgemm_small, every group size: one M tile with two column tiles per
    block where they fit (M = 24, N = 8400: 263 column tiles), two M tiles
    likewise (M = 64) and two M tiles with one column tile (M = 40, N =
    2000)."""
    xd = BF16 if sbd == BF16 else F16
    for gs in GROUPS:
        for M, N in [(24, 8400), (64, 8400), (40, 2000)]:
            name = f"small gemm b{bits} g{gs} sb{sbd} M{M} N{N}"
            _repeat(ctx, M, 1024, N, gs, bits, xd, sbd, "qgemm_small_kernel", name, 9000 + 7 * bits + M + gs)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("sbd", SB, ids=["sb_f16", "sb_bf16", "sb_f32"])
def test_mid_gemv_rings_repeat(ctx, bits, sbd):
    """qgemv_mid (M = 9..16 rows of x), every group size, K = 1024 and
    4096."""
    xd = BF16 if sbd == BF16 else F16
    for gs in GROUPS:
        for M, K in [(9, 1024), (16, 1024), (12, 4096)]:
            name = f"mid gemv b{bits} g{gs} sb{sbd} M{M} K{K}"
            _repeat(ctx, M, K, 4100, gs, bits, xd, sbd, "qgemv_mid_kernel", name, 9500 + 5 * bits + M + gs)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("sbd", SB, ids=["sb_f16", "sb_bf16", "sb_f32"])
def test_rw_gemm_repeat(ctx, bits, sbd):
    """qgemm_rw, every group size: 30 tiles in K parts meeting in the
    workspace (M = 640, N = 1536, fp32 out), and 264 tiles on the persistent
    grid, the last round's 8 tiles in K halves (M = 1024, N = 8448, 16-bit
    out); K = 2048."""
    xd = BF16 if sbd == BF16 else F16
    for gs in GROUPS:
        for M, N, od in [(640, 1536, F32), (1024, 8448, xd)]:
            name = f"rw gemm b{bits} g{gs} sb{sbd} M{M} N{N}"
            _repeat(ctx, M, 2048, N, gs, bits, xd, sbd, "qgemm_rw_kernel", name, 9700 + bits + M + gs, od=od,
                    launches=12)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sbd", SB, ids=["sb_f16", "sb_bf16", "sb_f32"])
def test_split_k_and_lds_gemm_repeat(ctx, bits, sbd):
    """qgemm_sk (M = 40, K = 3200: K % 1024 != 0, K parts) for every width,
    and qgemm_kernel (M = 384, K = 1024, N = 1280) for the widths the
    register-W GEMM does not take; every group size."""
    from mlx_amd import abi
    xd = BF16 if sbd == BF16 else F16
    for gs in GROUPS:
        _repeat(ctx, 40, 3200, 6000, gs, bits, xd, sbd, "qgemm_sk_kernel", f"split-K gemm b{bits} g{gs} sb{sbd}",
                9800 + bits + gs, launches=12)
        if bits in (4, 8) or ctx.kernel_name(384, 1024, 1280, gs, bits, xd, sbd, F32, abi.KERNEL_GEMM) is None:
            continue  # 4/8-bit: the register-W GEMM; none: no GEMM form (6-bit, f32 scales, group 32)
        _repeat(ctx, 384, 1024, 1280, gs, bits, xd, sbd, "qgemm_kernel", f"lds gemm b{bits} g{gs} sb{sbd}",
                9900 + bits + gs, launches=12)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sbd", SB, ids=["sb_f16", "sb_bf16", "sb_f32"])
def test_gemv_repeat(ctx, bits, sbd):
    """The GEMV kernels AUTO picks for M = 1..8 (whole-line, split-K,
    decode, 4x4x4-MFMA, K-split whole-line, stream and skinny kernels, and
    rows split over launches; several stage x or partial sums in LDS behind
    barriers), group
    sizes 32 and 128, K = 4096 and 14336, ragged N = 4100."""
    xd = BF16 if sbd == BF16 else F16
    for gs in (32, 128):
        for K in (4096, 14336):
            for M in (1, 2, 3, 4, 6, 8):
                _repeat(ctx, M, K, 4100, gs, bits, xd, sbd, None, f"gemv b{bits} g{gs} sb{sbd} M{M} K{K}",
                        9600 + bits + gs + M + K, launches=12)
