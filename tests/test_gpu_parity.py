"""GPU parity: the HIP plugin, called through its C ABI, against the CPU
oracle on the same seeded inputs.

Bit-exact: dequantize (fp32 output), quantize (codes, scales, biases).
Tolerance (qmm_util): quantized matmul on every kernel path.
Full BASELINE shapes: exact comparison for the decode/crossover/irregular
configs; the prefill GEMM (M=2048) is checked on a seeded sample of rows,
which the oracle finishes in seconds.
"""
import numpy as np
import pytest

from qmm_util import BF16, F16, F32, check_output

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 5, 6, 8]
KERNELS = {"auto": 0, "gemv": 1, "gemm": 2}


def run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, kernel=0):
    from mlx_amd import runtime
    print(f"[case] qmm M={M} K={K} N={N} g={gs} bits={bits} x={xd} sb={sbd} out={od} kernel={kernel}",
          flush=True)
    return runtime.run_quantized_matmul(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, kernel)


def test_device_and_buffers(ctx):
    info = ctx.device_info()
    assert b"gfx950" in info.name and info.is_discrete and not info.is_unified_memory
    assert info.compute_units >= 200 and info.memory_total > 100 * 2**30
    # buffer_alloc zero-fills; copies move min(bytes, size) bytes
    buf = ctx.alloc(64)
    assert np.all(buf.download(np.uint8, (64,)) == 0)
    big = np.arange(100, dtype=np.uint8)
    buf.upload(big)                       # 100 bytes into a 64-byte buffer
    out = np.full(80, 7, np.uint8)
    from mlx_amd import runtime
    runtime._check(ctx.vt.buffer_copy_to_host(ctx.handle, buf.handle, out.ctypes.data, 80), "copy")
    assert np.array_equal(out[:64], big[:64]) and np.all(out[64:] == 7)
    buf.free()
    ctx.sync()


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sb", [F32, F16, BF16])
def test_dequantize_bit_exact(ctx, oracle, bits, sb):
    from mlx_amd import runtime
    O = oracle
    N, K, gs = 37, 512, 64 if bits != 8 else 128
    w = O.rng_normal(N * K, 500 + bits, 0.0, 0.02).reshape(N, K)
    w_q, s, b = O.quantize(w, gs, bits, sb)
    for od in (F32, F16, BF16):
        print(f"[case] dequant bits={bits} sb={sb} out={od}", flush=True)
        got = runtime.run_dequantize(ctx, w_q, s, b, K, gs, bits, sb, od)
        want = O.dequantize(w_q, s, b, K, gs, bits, sb, od)
        assert np.array_equal(got.view(np.uint16 if od else np.uint32),
                              want.view(np.uint16 if od else np.uint32))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_bit_exact(ctx, oracle, bits, gs):
    """Codes, scales and biases bit-equal to the CPU quantizer, for f32 and
    16-bit weights, a partial last wave (N K / 8 not a multiple of 64), and
    the cases the parallel min/max must order like the sequential scan: a
    NaN first weight poisons its group, later NaNs are skipped, ties between
    -0 and +0 keep the first, an infinite weight."""
    from mlx_amd import runtime
    O = oracle
    N, K = 29, 512
    w = O.rng_normal(N * K, 900 + bits, 0.0, 0.02).reshape(N, K)
    w[0, :gs] = -0.5  # constant group
    w.reshape(-1)[::97] *= 20.0  # outliers
    w[1, gs] = np.nan             # first weight of group 1: the group is NaN
    w[1, 2 * gs + 5] = np.nan     # a later weight: skipped
    w[2, :gs] = 0.0               # mixed-sign zeros: the first occurrence wins
    w[2, 1:gs:3] = -0.0
    w[3, 3 * gs + 7] = np.inf
    for wd in (F32, F16, BF16):
        wi = w if wd == F32 else O.from_f32(w, wd)
        wf = w if wd == F32 else O.to_f32(wi, wd)
        for sb in (F32, F16, BF16):
            print(f"[case] quantize bits={bits} g={gs} w={wd} sb={sb}", flush=True)
            gq, gs_, gb = runtime.run_quantize(ctx, wi, gs, bits, wd, sb)
            wq, s, b = O.quantize(wf, gs, bits, sb)
            u = np.uint32 if sb == F32 else np.uint16
            assert np.array_equal(gq, wq)
            assert np.array_equal(gs_.view(u), s.view(u)) and np.array_equal(gb.view(u), b.view(u))


# ---- GEMV ---------------------------------------------------------------

@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_q4_two_chunk_parity(ctx, oracle, xd, sbd, od):
    """4-bit codes, M = 2..4, 8192 < K <= 16384: the 4x4x4-MFMA
    decode kernel with two 512-code chunks per lane on 12, 14 or 16 waves
    (each chunk with its own group factors), 16-row blocks with a ragged
    last one, every group size; K below the waves' reach leaves lanes past K
    idle: half of the last chunk's lanes (K = 11008), a whole last chunk (K
    = 13824), whole waves (K = 9216), all of waves 8..11 but two 32-code
    blocks of wave 8's first chunk (K = 8256)."""
    O = oracle
    for i, (K, N, gs) in enumerate([(12288, 300, 64), (14336, 77, 32), (16384, 130, 128), (14336, 4100, 64),
                                    (12288, 33, 32), (16384, 60, 64), (11008, 301, 64), (13824, 70, 128),
                                    (9216, 45, 32), (11008, 96, 32), (10240, 20, 128), (15360, 50, 64),
                                    (8256, 40, 32)]):
        M = 2 + i % 3
        assert ctx.kernel_name(M, K, N, gs, 4, xd, sbd, od) == "qgemv_q4_kernel"
        x, w_q, s, b, _ = O.make_problem(M, K, N, 4, gs, xd, sbd, seed=7300 + M + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od)
        check_output(O, y, want, od, f"q4 two chunks M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_row_split_long_k_parity(ctx, oracle, xd, sbd, od):
    """M = 5..8, 8192 < K <= 16384 where the LDS-ring kernel does not take
    the shape (K % 1024 != 0, 2-bit codes) or fills half the CUs (4-bit, N
    <= 4096): rows 0..3 and the rest of x as two launches of the M <= 4
    kernels (the two-chunk decode kernel for 4-bit codes, the K-split
    whole-line kernel for 2 and 8; a fifth row on the M = 1 kernels), each
    writing its own rows of y."""
    O = oracle
    for (M, K, N, bits, gs) in [(5, 11008, 301, 4, 64), (6, 14336, 200, 4, 32), (8, 11008, 96, 8, 32),
                                (7, 14336, 130, 2, 128), (5, 9216, 64, 2, 32), (8, 13824, 77, 4, 128),
                                (6, 10752, 45, 8, 64)]:
        assert ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od) in ("qgemv_q4_kernel", "qgemv_mx_kernel")
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=7600 + M + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"row split M{M} K{K} N{N} b{bits} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_split_k_row_pairs_parity(ctx, oracle, xd, sbd, od):
    """16-bit x, K > 4096, M = 3..8 where no M-wide kernel takes the shape
    (3/5/6-bit codes; K % 1024 != 0 for 4/8-bit; K up to 32768): pairs of
    rows on the split-K kernel, a last single
    row on the M = 1 split-K kernel, each launch writing its own rows of y;
    K up to 32768, ragged N, every group size."""
    O = oracle
    for (M, K, N, bits, gs) in [(3, 5120, 130, 3, 64), (4, 6144, 77, 5, 32), (5, 28672, 40, 6, 128),
                                (8, 4160, 33, 8, 64), (7, 6656, 50, 4, 128), (6, 32768, 20, 2, 64),
                                (3, 28672, 64, 3, 64)]:
        assert ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od) == "qgemv_split_kernel"
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=7800 + M + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"split-K row pairs M{M} K{K} N{N} b{bits} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_stream_row_chunks_parity(ctx, oracle, xd, sbd, od):
    """16-bit x, K <= 4096, M = 5..8 where no M-wide kernel takes the shape:
    chunks of 4 rows on the stream kernel (the last chunk 1..4 rows), each
    launch writing its own rows of y; ragged N, every group size."""
    O = oracle
    for (M, K, N, bits, gs) in [(5, 2048, 130, 3, 64), (8, 1024, 77, 6, 32), (6, 3072, 40, 5, 128),
                                (8, 2560, 33, 4, 64), (7, 512, 64, 2, 32), (6, 1536, 50, 8, 128)]:
        assert ctx.kernel_name(M, K, N, gs, bits, xd, sbd, od) == "qgemv_stream_kernel"
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=7900 + M + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"stream row chunks M{M} K{K} N{N} b{bits} g{gs}")


@pytest.mark.parametrize("sbd,od", [(F32, F32), (F16, F32), (BF16, F16), (F32, BF16)])
def test_f32_x_per_row_parity(ctx, oracle, sbd, od):
    """f32 x with 3/5/6-bit codes, M = 2..8, K <= 4096: one launch of the
    M = 1 kernels per row of x (whole-line for 3/6-bit, stream for 5-bit),
    each writing its own row of y; ragged N, every group size, K = 960 (an
    odd chunk count)."""
    O = oracle
    for (M, K, N, bits, gs) in [(2, 4096, 300, 3, 64), (3, 2048, 130, 5, 32), (4, 4096, 77, 6, 128),
                                (8, 1024, 96, 3, 32), (5, 4096, 40, 5, 64), (7, 960, 33, 6, 64),
                                (6, 4096, 1030, 6, 32)]:
        assert ctx.kernel_name(M, K, N, gs, bits, F32, sbd, od) in ("qgemv_line_kernel", "qgemv_stream_kernel")
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, F32, sbd, seed=7700 + M + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, F32, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F32, sbd, od)
        check_output(O, y, want, od, f"f32 x per row M{M} K{K} N{N} b{bits} g{gs}")


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_line_gemv_six_rows(ctx, oracle, bits, xd, sbd, od):
    """M = 1 on the whole-line GEMV where 2- to 4-bit codes with 16-bit x
    take 6-row waves (24-row blocks leave the busiest CU the fewest rows):
    N = 5120 (214 blocks, one per CU), 11000 (459 blocks, the last one
    ragged), 12288 (512 blocks, two per CU) and 5130 at K = 960 (an odd
    chunk count), every group size."""
    O = oracle
    for (K, N, gs) in [(4096, 5120, 64), (2048, 11000, 32), (4096, 12288, 128), (960, 5130, 32)]:
        assert ctx.kernel_name(1, K, N, gs, bits, xd, sbd, od) == "qgemv_line_kernel"
        x, w_q, s, b, _ = O.make_problem(1, K, N, bits, gs, xd, sbd, seed=bits * 53 + N)
        y = run(ctx, x, w_q, s, b, 1, K, N, gs, bits, xd, sbd, od)
        want = O.quantized_matmul(x, w_q, s, b, 1, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"line six rows b{bits} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F32, F32, F32),
                                       (F16, F32, F32), (BF16, F16, F32)])
def test_gemv_parity(ctx, oracle, bits, xd, sbd, od):
    O = oracle
    # M = 1 with K <= 4096 runs the whole-line kernel: full and partial last
    # wave loads, an odd chunk count (K = 960), group sizes 32/64/128 (2-bit
    # codes with group size 32: two groups per chunk), ragged N
    for (M, K, N, gs) in [(1, 4096, 300, 64), (1, 960, 77, 32), (1, 2048, 129, 128), (1, 192, 17, 32),
                          (3, 1024, 129, 32), (8, 512, 77, 128), (5, 8192, 64, 64), (2, 192, 33, 64)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 31 + M)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"gemv b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F32, F32, F32),
                                       (F16, F32, F32), (BF16, F16, F32)])
def test_split_k_gemv_parity(ctx, oracle, bits, xd, sbd, od):
    """M = 1 with 4096 < K <= 32768 (and M = 2 with 16-bit x and
    8192 < K <= 16384) runs the split-K stream kernel: parts of
    64 units (K = 8192: 2 waves), uneven parts with idle lanes (K = 5120:
    2 x 40 units; K = 14336: 4 x 56), 7 and 8 waves (K = 28672, 32768; f32
    x at K = 32768 exceeds its LDS and runs the generic kernel), every group
    size, N not a multiple of the 4-row block.  fp32 outputs with K > 8192
    meet the fp32 gate (1e-5 of max|y|) against the oracle's fp64
    accumulation: over that many terms the sequential fp32 oracle's own
    rounding reaches ~1e-5 (measured 1.3e-5 between it and this kernel at
    K = 14336)."""
    O = oracle
    # (1, 28672, 11, 32): f32 x and scales need the 4-row block form there
    # (8 rows of g32 f32 scales do not fit next to 112 KB of x); (2, 12288,
    # 13, 32) and (2, 14336, 21, 64) run the two-row form on both x rows;
    # (1, 5120, 23, 32) and (1, 14336, 19, 32): idle lanes (masked scales)
    # with two groups per unit
    for (M, K, N, gs) in [(1, 5120, 37, 128), (1, 8192, 50, 32), (1, 14336, 21, 64), (1, 28672, 13, 64),
                          (1, 28672, 11, 32), (1, 32768, 9, 32), (2, 14336, 21, 64), (2, 9216, 13, 128),
                          (2, 12288, 13, 32), (2, 16384, 6, 32), (1, 5120, 23, 32), (1, 14336, 19, 32)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 17 + K + M)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemv"])
        if od == F32 and K > 8192:
            want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="f64").astype(np.float32)
        else:
            want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"split-K b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("K,N,xd", [(14336, 4096, F16), (28672, 8192, BF16)])
def test_split_k_full(ctx, oracle, K, N, xd):
    """Model-sized M = 1 shapes on the split-K kernel: a down projection
    (K = 14336, N = 4096) and K = 28672, N = 8192; 4-bit g64."""
    O = oracle
    x, w_q, s, b, _ = O.make_problem(1, K, N, 4, 64, xd, xd, seed=K + N)
    y = run(ctx, x, w_q, s, b, 1, K, N, 64, 4, xd, xd, xd)
    want = O.quantized_matmul(x, w_q, s, b, 1, K, N, 64, 4, xd, xd, xd, variant="omp")
    check_output(O, y, want, xd, f"split-K full K{K} N{N}")


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_kline_gemv_parity(ctx, oracle, bits, xd, sbd, od):
    """2 <= M <= 4 rows of x with K <= 4096 (K % 256 == 0, each quarter of K
    a whole number of groups) runs the K-split whole-line kernel where it is
    the faster one: 8-bit codes at M = 2..4, 2-bit at M = 3 and 4, 4-bit at
    M = 2 with f16 x (the other cases check the kernels that take them).
    M = 3 carries a fourth x row that is never stored; 16- and 28-row blocks
    (N = 7150: 256 blocks of 28, the last ragged); a quarter of K narrower
    than a wave (K = 256: 4 of 64 lanes hold codes); every group size."""
    O = oracle
    Ms = {2: (3, 4), 4: (2,), 8: (2, 3, 4)}[bits]
    shapes = [(Ms[i % len(Ms)], K, N, gs) for i, (K, N, gs) in
              enumerate([(4096, 300, 64), (1024, 77, 32), (2048, 129, 128), (256, 40, 64), (512, 57, 128),
                         (4096, 7150, 32)])]
    for (M, K, N, gs) in shapes:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 41 + M + K)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"k-line b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32),
                                       (F16, BF16, F32)])
def test_q4_decode_parity(ctx, oracle, xd, sbd, od):
    """2 <= M <= 8 rows of x with 4-bit codes and K = 2048, 4096 or 8192 run
    the 4x4x4-MFMA decode kernel: one and two sets of 4 x rows (M = 5..7
    carry x rows that are never stored), 4, 8 and 16 waves, 16- and 28-row
    blocks (N = 7150: 256 blocks of 28, the last ragged), every group size,
    N not a multiple of the 4-row group."""
    O = oracle
    for (M, K, N, gs) in [(2, 4096, 300, 64), (3, 2048, 77, 32), (4, 8192, 130, 128), (5, 4096, 33, 32),
                          (6, 2048, 7150, 64), (7, 8192, 41, 64), (8, 4096, 7150, 128), (8, 2048, 19, 32),
                          (4, 4096, 14336, 64)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, 4, gs, xd, sbd, seed=M * 53 + K + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od)
        check_output(O, y, want, od, f"q4 M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sbd,od", [(F32, F32), (F16, F32), (BF16, F16)])
def test_kline_gemv_f32_x(ctx, oracle, bits, sbd, od):
    """f32 x at 2 <= M <= 4: the K-split whole-line kernel takes every K it
    applies to (K <= 16384, each wave's part a whole number of 16-code
    chunks), with 4, 8 and 16 waves per block and, at 16 waves, half the
    rows of the 16-bit x blocks (f32 x is 16 VGPRs per row of x); M = 5..9
    in chunks of 4 rows (a last single row on the M = 1 kernels).  fp32
    outputs with K > 8192 are gated against the oracle's fp64 accumulation
    (the sequential fp32 oracle's own rounding reaches ~1e-5 there)."""
    O = oracle
    for i, (K, N, gs) in enumerate([(4096, 300, 64), (1024, 77, 32), (256, 40, 64), (2048, 7150, 128),
                                    (6144, 100, 64), (8192, 33, 32), (14336, 70, 32), (16384, 19, 128),
                                    (4096, 130, 64), (14336, 33, 128), (2048, 65, 32)]):
        M = 2 + (i + bits) % 3 if i < 8 else (5, 8, 9)[i - 8]
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, F32, sbd, seed=bits * 47 + M + K)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, F32, sbd, od, KERNELS["gemv"])
        if od == F32 and K > 8192:
            want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F32, sbd, od, variant="f64").astype(np.float32)
        else:
            want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F32, sbd, od)
        check_output(O, y, want, od, f"k-line f32 x b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_small_m_mfma_parity(ctx, oracle, bits, xd, sbd, od):
    """2 <= M <= 16 with 4/8-bit codes: the MFMA kernels (for K % 1024 == 0
    the decode kernel at M <= 8 with 4-bit codes, else the LDS-ring one; the
    skinny one for other K), and the launcher's exceptions to them: M = 2
    with K <= 4096 runs the stream kernel, 8-bit codes with M <= 8 and
    K <= 4096 the stream (M <= 4) or skinny kernels (the LDS-ring kernel
    keeps M = 4, K = 6144).  Every group size, one and two x DMAs per step,
    row tails in the 16-row tile and in the 32-column block."""
    O = oracle
    for (M, K, N, gs) in [(2, 1024, 77, 32), (4, 2048, 50, 64), (5, 1024, 77, 32), (8, 2048, 50, 64),
                          (4, 6144, 37, 64),
                          (16, 4096, 40, 128), (6, 4096, 33, 64), (12, 4096, 21, 32), (3, 3072, 65, 128),
                          (9, 1024, 96, 64), (7, 512, 40, 64), (10, 256, 19, 32)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 7 + M)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"small-M b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_kline_gemv_long_k(ctx, oracle, bits, xd, sbd, od):
    """2 <= M <= 4 with 4096 < K <= 16384 (down projections): the K-split
    whole-line kernel with 8 waves per block (4096 < K <= 8192, where it takes
    M = 2 and 2-bit codes) and 16 (K <= 16384, every M), each wave's part
    under a whole wave (K = 6144: 768 codes, 48 lanes), every group size, f32
    scales whose block rows take two LDS passes (K = 16384, g32), ragged N;
    4-bit codes at K = 12288 / 14336 / 16384 run the 4x4x4-MFMA decode kernel
    with two chunks per lane instead."""
    O = oracle
    for i, (K, N, gs) in enumerate([(6144, 100, 64), (8192, 33, 32), (14336, 70, 32), (16384, 40, 128),
                                    (16384, 18, 32), (12288, 50, 64)]):
        M = (2 if bits != 2 else 3) if K <= 8192 else 2 + i % 3
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 43 + M + K)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od)
        check_output(O, y, want, od, f"k-line long K b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32),
                                       (F16, BF16, F32), (BF16, F32, BF16)])
def test_decode_mfma_parity(ctx, oracle, xd, sbd, od):
    """2 <= M <= 8 with 4-bit codes and K % 1024 == 0 runs the MFMA decode
    kernel (M <= 4 only for K > 4096, M = 2 only for 4096 < K <= 8192):
    every group size (all three lane regroupings), one to eight K waves, N
    not a multiple of the 32-row block, M at both ends.  f32 scales with
    group size 32 fall back to the LDS-ring kernel."""
    O = oracle
    for (M, K, N, gs) in [(2, 6144, 45, 64), (8, 4096, 100, 64), (3, 8192, 77, 32), (7, 8192, 33, 128),
                          (4, 5120, 64, 32), (6, 3072, 19, 128), (5, 1024, 128, 64), (8, 8192, 50, 32)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, 4, gs, xd, sbd, seed=11 * M + gs)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od)
        check_output(O, y, want, od, f"decode M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_decode_block_shapes(ctx, oracle, xd, sbd, od):
    """The decode launcher's two block shapes: 2-tile blocks when N/32 > 256
    (N = 8208 and 8200: a half-empty last tile and a partly empty one), or
    when the 1-tile blocks would not all be resident (M = 8, K = 8192: one
    block fills a CU's LDS); 1-tile blocks otherwise (N = 8192, M = 4,
    K = 8192: 512 blocks of 8 waves, two per CU)."""
    O = oracle
    for (M, K, N, gs) in [(3, 1024, 8208, 32), (8, 2048, 8200, 64), (8, 8192, 8192, 128), (4, 8192, 8192, 64)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, 4, gs, xd, sbd, seed=13 * M + gs)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od, KERNELS["gemv"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, 4, xd, sbd, od, variant="omp")
        check_output(O, y, want, od, f"decode blocks M{M} K{K} N{N} g{gs}")


def test_gemv_is_deterministic(ctx, oracle):
    O = oracle
    x, w_q, s, b, _ = O.make_problem(4, 4096, 512, 4, 64, F16, F16, seed=5)
    y1 = run(ctx, x, w_q, s, b, 4, 4096, 512, 64, 4, F16, F16, F32, 1)
    y2 = run(ctx, x, w_q, s, b, 4, 4096, 512, 64, 4, F16, F16, F32, 1)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_generic_path_for_odd_k(ctx, oracle):
    """K not a multiple of 64 (group 32) runs the generic kernel, which
    accumulates in the oracle's order: bit-exact fp32."""
    O = oracle
    for K in (32, 96, 160):
        x, w_q, s, b, _ = O.make_problem(3, K, 21, 3, 32, F32, F32, seed=K)
        y = run(ctx, x, w_q, s, b, 3, K, 21, 32, 3, F32, F32, F32)
        want = O.quantized_matmul(x, w_q, s, b, 3, K, 21, 32, 3, F32, F32, F32)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


# ---- full BASELINE shapes -----------------------------------------------

@pytest.mark.parametrize("M", [1, 4, 8])
def test_config1_decode_full(ctx, oracle, M):
    """4-bit g64, K=4096, N=14336, fp16 x/scales/out."""
    O = oracle
    K, N = 4096, 14336
    x, w_q, s, b, _ = O.make_problem(M, K, N, 4, 64, F16, F16, seed=1000 + M)
    y = run(ctx, x, w_q, s, b, M, K, N, 64, 4, F16, F16, F16)
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, 4, F16, F16, F16, variant="omp")
    check_output(O, y, want, F16, f"config1 M={M}")


def test_config0_cpu_plumbing_full(ctx, oracle):
    """M=1, K=N=4096, 4-bit g64, fp32 everything: tolerance 1e-5."""
    O = oracle
    x, w_q, s, b, _ = O.make_problem(1, 4096, 4096, 4, 64, F32, F32, seed=0)
    y = run(ctx, x, w_q, s, b, 1, 4096, 4096, 64, 4, F32, F32, F32)
    want = O.quantized_matmul(x, w_q, s, b, 1, 4096, 4096, 64, 4, F32, F32, F32)
    check_output(O, y, want, F32, "config0")


@pytest.mark.parametrize("bits", [3, 6])
@pytest.mark.parametrize("M", [1, 64])
def test_config4_irregular_full(ctx, oracle, bits, M):
    """3/6-bit g64, K=4096, N=11008, 1% x20 outliers, fp16."""
    O = oracle
    K, N = 4096, 11008
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, 64, F16, F16, seed=2000 + bits,
                                     outlier_frac=0.01, outlier_scale=20.0)
    # unpack is bit-exact: dequantized weights equal the oracle's
    from mlx_amd import runtime
    rows = slice(0, 256)
    got = runtime.run_dequantize(ctx, w_q[rows], s[rows], b[rows], K, 64, bits, F16, F32)
    assert np.array_equal(got, O.dequantize(w_q[rows], s[rows], b[rows], K, 64, bits, F16, F32))
    from mlx_amd import abi
    gemm = ctx.select_kernel(M, K, N, 64, bits, F16) == abi.KERNEL_GEMM
    y = run(ctx, x, w_q, s, b, M, K, N, 64, bits, F16, F16, F16)
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, bits, F16, F16, F16, variant="omp",
                              w_round=F16 if gemm else F32)
    check_output(O, y, want, F16, f"config4 b{bits} M{M}")
    if gemm:
        # f16 weight rounding stays inside the f16 gate against the exact form too
        exact = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, bits, F16, F16, F16, variant="omp")
        check_output(O, y, exact, F16, f"config4 b{bits} M{M} vs exact")


def test_config2_crossover_full(ctx, oracle):
    """8-bit g128, M=32, K=N=8192, bf16."""
    O = oracle
    M, K, N = 32, 8192, 8192
    x, w_q, s, b, _ = O.make_problem(M, K, N, 8, 128, BF16, BF16, seed=3000)
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, BF16, variant="omp")
    want32 = O.quantized_matmul(x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, F32, variant="omp")
    wantT = O.quantized_matmul(x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, BF16, variant="omp",
                               w_round=BF16)
    wantT32 = O.quantized_matmul(x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, F32, variant="omp",
                                 w_round=BF16)
    from mlx_amd import abi
    sel = ctx.select_kernel(M, K, N, 128, 8, BF16)
    for kname, k in KERNELS.items():
        # the GEMM (and AUTO when it picks the GEMM) dequantizes to bf16 first
        gemm = k == abi.KERNEL_GEMM or (k == abi.KERNEL_AUTO and sel == abi.KERNEL_GEMM)
        ref, ref32 = (wantT, wantT32) if gemm else (want, want32)
        y = run(ctx, x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, BF16, k)
        r = check_output(O, y, ref, BF16, f"config2 {kname}")
        # the same kernel with an fp32 epilogue meets the fp32 gate
        y32 = run(ctx, x, w_q, s, b, M, K, N, 128, 8, BF16, BF16, F32, k)
        r32 = check_output(O, y32, ref32, F32, f"config2 {kname} fp32 out")
        print(f"config2 {kname}: bf16-out max|d|/max|y| = {r:.3g}, fp32-out = {r32:.3g}")


# ---- errors -------------------------------------------------------------

def test_error_codes(ctx, oracle):
    from mlx_amd import abi, runtime
    O = oracle
    x, w_q, s, b, _ = O.make_problem(1, 256, 8, 4, 64, F16, F16, seed=1)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    out = ctx.alloc(8 * 2)
    q = ctx.q

    def call(M=1, K=256, N=8, gs=64, bits=4, xd=F16, sbd=F16, od=F16, o=out):
        return q.op_quantized_matmul(ctx.handle, *[t.handle for t in bufs], o.handle, M, K, N, gs,
                                     bits, xd, sbd, od)
    assert call() == abi.OK
    assert call(bits=7) == abi.ERR_NOT_SUPPORTED
    assert call(gs=48) == abi.ERR_NOT_SUPPORTED
    assert call(xd=abi.INT32) == abi.ERR_NOT_SUPPORTED
    assert call(K=250) == abi.ERR_INVALID_ARGUMENT       # K % group
    assert call(N=9) == abi.ERR_INVALID_ARGUMENT         # buffers too small for the shape
    assert call(M=-1) == abi.ERR_INVALID_ARGUMENT
    assert call(M=0) == abi.OK and call(N=0) == abi.OK   # empty problems are no-ops
    small = ctx.alloc(4)
    assert call(o=small) == abi.ERR_INVALID_ARGUMENT
    assert q.op_quantized_matmul_ex(ctx.handle, *[t.handle for t in bufs], out.handle, 1, 256, 8,
                                    64, 4, F32, F16, F16, abi.KERNEL_GEMM) in (
                                        abi.ERR_NOT_SUPPORTED, abi.ERR_INVALID_ARGUMENT)
    ctx.sync()
    for t in bufs + [out, small]:
        t.free()
    runtime._check(abi.OK, "ok")


# ---- GEMM (dequantize to the activation type, MFMA) ----------------------

@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(BF16, BF16, BF16), (F16, F16, F16), (BF16, F32, F32),
                                       (F16, BF16, F32)])
def test_gemm_parity(ctx, oracle, bits, xd, sbd, od):
    """The GEMM equals the oracle's "dequantize to T, then matmul" form
    (w_round = x dtype) to the dtype gates; ragged M and N exercise the
    tile edges."""
    from mlx_amd import abi, runtime
    O = oracle
    for (M, K, N, gs) in [(300, 512, 200, 64), (256, 1024, 128, 32), (33, 256, 130, 128),
                          (512, 768, 384, 64)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 17 + M)
        if sbd == F32 and gs == 32 and bits >= 6 and not (bits == 8 and K % 1024 == 0):
            # the GEMM's LDS buffers do not fit one CU for this combination
            # (the register-W kernel takes 8-bit codes with K % 1024 == 0)
            with pytest.raises(runtime.LuxError) as e:
                run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
            assert e.value.code == abi.ERR_NOT_SUPPORTED
            assert ctx.select_kernel(M, K, N, gs, bits, xd, sbd) == abi.KERNEL_GEMV
            continue
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, w_round=xd)
        check_output(O, y, want, od, f"gemm b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("xd,sbd,od", [(BF16, BF16, BF16), (F16, F16, F16), (BF16, F32, F32),
                                       (F16, BF16, F32)])
def test_rw_gemm_parity(ctx, oracle, bits, gs, xd, sbd, od):
    """M > 64, 4/8-bit codes, K % 1024 == 0: the register-W GEMM (128 x 256
    tiles, each wave dequantizing its own columns' codes into its MFMA
    operand).  Against the oracle's dequantize-to-T form: ragged M and N
    (tile edges, rows and columns past the ends), a shape whose 128 tiles all
    run as two K halves meeting in the workspace, and one on the XCD-grouped
    tile order (16 x 16 tiles)."""
    O = oracle
    for (M, K, N) in [(300, 1024, 200), (513, 2048, 520), (1024, 2048, 4096), (2048, 1024, 4096)]:
        print(f"[case] rw gemm b{bits} g{gs} x{xd} s{sbd} o{od} M{M} K{K} N{N}", flush=True)
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 31 + M + gs)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="omp", w_round=xd)
        check_output(O, y, want, od, f"rw gemm b{bits} g{gs} M{M} K{K} N{N}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_small_gemm_parity(ctx, oracle, bits, xd, sbd, od):
    """8 < M <= 64 with K % 1024 == 0 runs the W-streaming small-M GEMM: the
    same "dequantize to T, then matmul" form as the large GEMM, one and two
    32-row M tiles, ragged M and N, every group size, 4/8/12 steps per wave."""
    O = oracle
    for (M, K, N, gs) in [(9, 1024, 77, 64), (32, 2048, 130, 128), (33, 1024, 40, 32),
                          (64, 1024, 96, 64), (48, 3072, 33, 32)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 13 + M)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, w_round=xd)
        check_output(O, y, want, od, f"small gemm b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, F32, F32)])
def test_small_gemm_two_tiles_parity(ctx, oracle, bits, xd, sbd, od):
    """Past 256 column tiles of 32 (N > 8192) the small-M GEMM runs two tiles
    per block where their rings fit (6- and 8-bit codes through half- or
    quarter-super-step W slots; 5-, 6- and 8-bit codes with f32 scales at
    group 32 and two M tiles keep one tile and run two rounds):
    ragged N with the last block's second tile wholly past N (N = 8200),
    group sizes 32 (the rings fill the 160 KB exactly for 4-bit codes with
    f32 scales and 8-bit ones with 16-bit scales), 64 and 128, one and two M
    tiles."""
    O = oracle
    for (M, K, N, gs) in [(64, 1024, 8200, 32), (17, 2048, 9000, 64), (40, 1024, 12345, 128),
                          (32, 1024, 8400, 32)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 7 + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="omp", w_round=xd)
        check_output(O, y, want, od, f"small gemm two tiles b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("xd,sbd,od", [(F16, F16, F16), (BF16, BF16, BF16), (F16, F32, F32), (BF16, F16, F32)])
def test_split_k_gemm_parity(ctx, oracle, bits, xd, sbd, od):
    """8 < M <= 64 with K % 128 == 0 and K % 1024 != 0: the split-K small-M
    GEMM, the GEMM form ("dequantize to T, then matmul").  The shapes take
    the K-part counts 1 (3 super-steps), 3 (of 9), 15 (of 30), 10 (of 20)
    and 31 (of 62), one and two M tiles, ragged M and N; the parts meet
    through the context's workspace."""
    O = oracle
    for (M, K, N, gs) in [(9, 384, 77, 32), (12, 1152, 200, 64), (40, 3840, 300, 128),
                          (64, 2560, 1000, 32), (17, 7936, 129, 64)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 31 + M)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, w_round=xd)
        check_output(O, y, want, od, f"split-K gemm b{bits} M{M} K{K} N{N} g{gs}")


@pytest.mark.parametrize("M,xd,sbd,od", [(33, F16, F16, F16), (64, BF16, BF16, F32), (16, BF16, F32, BF16)])
def test_unsplit_wide_gemm_parity(ctx, oracle, M, xd, sbd, od):
    """Wide N (>= 192 tiles of 128 columns) runs the same kernel unsplit,
    with no workspace: 193 tiles, the last one ragged (N = 24600)."""
    O = oracle
    K, N, gs, bits = 1024, 24600, 64, 4
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=610 + M)
    y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="omp", w_round=xd)
    check_output(O, y, want, od, f"unsplit wide M{M}")


def test_split_k_shapes_in_sequence(ctx, oracle):
    """Split-K GEMM launches of different shapes back to back on one
    context workspace: a shape with few tiles and large partials (8 tiles,
    14 K parts), then one with 188 tiles (2 K parts), then the first again.
    Every tile counter must read zero at the start of each launch, so no
    shape's partials may land on another's counter slots."""
    O = oracle
    A = (64, 3584, 1024, 4, 64)
    B = (64, 2560, 24000, 4, 64)
    for i, (M, K, N, bits, gs) in enumerate([A, B, A]):
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, BF16, BF16, seed=900 + N)
        y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, BF16, BF16, F32, KERNELS["gemm"])
        want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, BF16, BF16, F32, variant="omp", w_round=BF16)
        check_output(O, y, want, F32, f"split-K sequence launch {i} N={N}")


@pytest.mark.parametrize("M,K,N,bits,gs,xd,kern", [
    (32, 8192, 8192, 8, 128, BF16, "gemm"),   # small-M GEMM, one block per CU
    (64, 4096, 11008, 3, 64, F16, "gemm"),    # two M tiles, two column tiles per block, ragged grid
    (64, 4096, 11008, 6, 64, F16, "gemm"),    # the same with the 6-bit half-slot W ring
    (64, 4096, 11008, 8, 64, F16, "gemm"),    # the same with the 8-bit quarter-slot W ring
    (32, 8192, 16384, 4, 64, BF16, "gemm"),   # one M tile, two column tiles per block, 256 blocks
    (32, 4096, 14336, 8, 128, BF16, "gemm"),  # the same with the 8-bit half-slot W ring
    (16, 4096, 14336, 4, 64, BF16, "gemv"),   # mid-M GEMV rings
])
def test_ring_kernels_repeat_full_grid(ctx, oracle, M, K, N, bits, gs, xd, kern):
    """The per-wave DMA ring kernels over a full grid (every CU busy), six
    launches in a row: each equals the oracle and the first bit for bit.
    A ring slot refilled while a read of its previous contents was still
    queued once gave stale operands in a few blocks of such launches."""
    O = oracle
    from mlx_amd import abi
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, xd, seed=4000 + M)
    gemm = kern == "gemm"
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, xd, F32, variant="omp",
                              w_round=xd if gemm else F32)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    out = ctx.alloc(M * N * 4)
    try:
        first = None
        for rep in range(6):
            print(f"[case] ring repeat {rep} M={M} K={K} N={N} b={bits} kernel={kern}", flush=True)
            ctx.quantized_matmul(*bufs, out, M, K, N, gs, bits, xd, xd, F32,
                                 abi.KERNEL_GEMM if gemm else abi.KERNEL_GEMV)
            y = out.download(np.float32, (M, N))
            check_output(O, y, want, F32, f"ring repeat {rep}")
            if first is None:
                first = y
            assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), f"launch {rep} differs from launch 0"
    finally:
        for t in bufs + [out]:
            t.free()


@pytest.mark.parametrize("M,K,N,bits,gs,xd,sbd", [
    (32, 4096, 11008, 8, 32, BF16, F32),   # quarter-super-step W slots, three x slots
    (32, 4096, 11008, 8, 64, F16, F16),    # half-super-step W slots, three x slots
    (64, 4096, 11008, 8, 64, F16, F16),    # quarter-super-step W slots, two x slots
])
def test_small_gemm_first_steps_repeat(ctx, oracle, M, K, N, bits, gs, xd, sbd):
    """The two-tile small-M GEMM on part-super-step W slots over a full grid,
    48 launches in a row: the first equals the oracle and every one the first
    bit for bit.  The waits of a wave's first steps count the DMAs issued
    after its x as the steady state orders them; a prologue that issued every
    W unit ahead of x left the first step of the 8-bit, f32-scale, group-32
    tiles able to read x before it landed (4 to 12 distinct outputs in 64
    launches)."""
    O = oracle
    from mlx_amd import abi
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=4100 + M + gs)
    want = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32, variant="omp", w_round=xd)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    out = ctx.alloc(M * N * 4)
    try:
        print(f"[case] small gemm first steps M={M} K={K} N={N} b={bits} g={gs} s={sbd}", flush=True)
        first = None
        for rep in range(48):
            ctx.quantized_matmul(*bufs, out, M, K, N, gs, bits, xd, sbd, F32, abi.KERNEL_GEMM)
            y = out.download(np.float32, (M, N))
            if first is None:
                check_output(O, y, want, F32, "small gemm first steps")
                first = y
            assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), f"launch {rep} differs from launch 0"
    finally:
        for t in bufs + [out]:
            t.free()


def test_gemm_shape_limits(ctx, oracle):
    """K not a multiple of 256: an explicit GEMM request is NOT_SUPPORTED,
    AUTO picks the GEMV (exact weights) for any M."""
    from mlx_amd import abi
    O = oracle
    M, K, N = 64, 192, 40
    assert ctx.select_kernel(M, K, N, 64, 4, F16) == abi.KERNEL_GEMV
    assert ctx.select_kernel(M, 256, N, 64, 4, F16) == abi.KERNEL_GEMM
    assert ctx.select_kernel(M, 256, N, 64, 4, F32) == abi.KERNEL_GEMV
    x, w_q, s, b, _ = O.make_problem(M, K, N, 4, 64, F16, F16, seed=5)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    out = ctx.alloc(M * N * 4)
    rc = ctx.q.op_quantized_matmul_ex(ctx.handle, *[t.handle for t in bufs], out.handle, M, K, N,
                                      64, 4, F16, F16, F32, abi.KERNEL_GEMM)
    assert rc == abi.ERR_NOT_SUPPORTED
    ctx.sync()
    for t in bufs + [out]:
        t.free()
    y = run(ctx, x, w_q, s, b, M, K, N, 64, 4, F16, F16, F32)
    check_output(O, y, O.quantized_matmul(x, w_q, s, b, M, K, N, 64, 4, F16, F16, F32), F32,
                 "auto K=192")


@pytest.mark.parametrize("N", [4096, 14336])
def test_config3_prefill(ctx, oracle, N):
    """M=2048, K=4096, 4-bit g64, bf16.  The whole output (all
    2048 rows, both N) is computed on the GPU and checked against the oracle
    (the dequantize-to-bf16 form, bf16 and fp32 outputs; the bf16 form is
    the oracle's fp32 sums rounded RNE, as the oracle's bf16 output is).
    The deviation from the exact fp32-weight form is bounded too: the bf16
    rounding of the weights (2^-9 relative each) measured 1.5e-3 of max|y|
    with fp32 outputs; a bf16 output adds up to one bf16 ulp of the largest
    value (2^-8 relative)."""
    O = oracle
    M, K = 2048, 4096
    print(f"[case] config3 M={M} K={K} N={N}", flush=True)
    x, w_q, s, b, _ = O.make_problem(M, K, N, 4, 64, BF16, BF16, seed=4000 + N)
    want32 = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, 4, BF16, BF16, F32, variant="omp",
                                w_round=BF16)
    exact = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, 4, BF16, BF16, F32, variant="omp")
    for od in (BF16, F32):
        y = run(ctx, x, w_q, s, b, M, K, N, 64, 4, BF16, BF16, od)
        want = want32 if od == F32 else O.from_f32(want32, BF16)
        r = check_output(O, y, want, od, f"config3 N={N} out={od}")
        g = O.to_f32(y, od) if od != F32 else y
        dev = float(np.abs(g - exact).max() / np.abs(exact).max())
        print(f"config3 N={N} out={od}: vs dequant-to-bf16 oracle {r:.3g}, vs exact-weight oracle {dev:.3g}")
        assert dev < (2.5e-3 if od == F32 else 2.5e-3 + 2.0 ** -8)


def test_gemm_split_last_round(ctx, oracle):
    """The large GEMM runs a last round that is at most half full as two K
    halves per tile, meeting in the context's workspace: 16 tiles (all
    split), then 264 tiles (the last 8 split: one column of tiles, all M
    tiles), then the first shape again.  Each tile counter must be back at
    zero after its launch, and a split result equals the oracle's
    dequantize-to-bf16 form as the unsplit tiles do; the first shape's
    repeat is bit-identical to its first run."""
    O = oracle
    A = (512, 1024, 1024)
    B = (2048, 512, 4224)
    first = None
    for i, (M, K, N) in enumerate([A, B, A]):
        print(f"[case] split last round launch {i} M={M} K={K} N={N}", flush=True)
        x, w_q, s, b, _ = O.make_problem(M, K, N, 4, 64, BF16, BF16, seed=950 + N)
        y = run(ctx, x, w_q, s, b, M, K, N, 64, 4, BF16, BF16, F32, KERNELS["gemm"])
        rows = np.arange(M) if M <= 512 else np.sort(np.random.default_rng(N).choice(M, 64, replace=False))
        xs = np.ascontiguousarray(x[rows])
        want = O.quantized_matmul(xs, w_q, s, b, len(rows), K, N, 64, 4, BF16, BF16, F32, variant="omp",
                                  w_round=BF16)
        check_output(O, np.ascontiguousarray(y[rows]), want, F32, f"split last round launch {i} N={N}")
        if (M, K, N) == A:
            if first is None:
                first = y
            else:
                assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), "repeat differs"


PERSISTENT_CASES = [
    # M, K, N, bits, gs, x, scales: more 128 x 256 tiles than CUs with a
    # 16-bit output, so one block per CU runs several units in turn
    (2000, 1024, 4360, 4, 64, BF16, BF16),   # 288 tiles: 64 blocks go on from a whole tile to a K half
    (1000, 2048, 16136, 8, 128, F16, F16),   # 512 tiles, two per block; 8-bit: staged in the rings
    (2048, 1024, 8200, 4, 32, F16, F32),     # 512 tiles + 16 split; f32 scales
]


@pytest.mark.parametrize("case", PERSISTENT_CASES, ids=lambda c: f"M{c[0]}K{c[1]}N{c[2]}b{c[3]}")
def test_rw_gemm_persistent_parity(ctx, oracle, case):
    """The register-W GEMM on one block per CU, each block running units b,
    b + 256, ...: a finished tile is staged and stored while the next
    unit's first transfers land.  Whole outputs against the oracle's
    dequantize-to-T form: ragged M (the last M tile's rows past M are
    dropped by offset), ragged N (N % 256 != 0), the hand-over into a split
    K half, both 16-bit outputs, and the fused output stage (bias and
    activation applied in the hand-over's staging)."""
    from mlx_amd import runtime
    O = oracle
    M, K, N, bits, gs, xd, sbd = case
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=7100 + N)
    acc = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32, variant="omp", w_round=xd)
    od = xd
    y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, KERNELS["gemm"])
    check_output(O, y, O.from_f32(acc, od), od, f"persistent M{M} N{N} out{od}")
    bias = O.from_f32(O.rng_normal(N, seed=7200 + N), F32)
    act = 2 if bits == 4 else 3  # silu / gelu
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    bb = ctx.upload(bias)
    try:
        out = ctx.alloc(M * N * runtime.esize(od))
        print(f"[case] persistent fused M={M} K={K} N={N} act={act} out={od}", flush=True)
        ctx.quantized_matmul_fused(*bufs, bb, out, M, K, N, gs, bits, xd, sbd, F32, od, act)
        yf = out.download(runtime.np_dtype(od), (M, N))
        out.free()
        check_output(O, yf, O.fused_epilogue(acc, bias, F32, act, od), od, f"persistent fused act{act}")
    finally:
        for t in bufs + [bb]:
            t.free()


# ---- fused output stage (bias + activation in the kernel's store) ---------

FUSED_CASES = [
    # M, K, N, bits, gs, x dtype: AUTO routes each to a different kernel
    (1, 4096, 300, 4, 64, F16),     # whole-line GEMV
    (1, 4096, 5120, 3, 64, BF16),   # whole-line GEMV, 6-row waves
    (1, 14336, 70, 4, 64, BF16),    # split-K GEMV
    (3, 5120, 40, 5, 64, BF16),     # split-K GEMV on pairs of rows (5-bit, three rows of x)
    (3, 14336, 72, 4, 64, F16),     # 4x4x4-MFMA decode, two chunks per lane
    (6, 11008, 72, 4, 64, BF16),    # rows 0..3 and 4..5 as two launches (two-chunk decode)
    (2, 4096, 40, 4, 64, F16),      # K-split whole-line GEMV (two rows of x)
    (2, 4096, 40, 3, 64, F16),      # stream GEMV (two rows of x, 3-bit)
    (6, 960, 70, 3, 64, F16),       # stream GEMV in chunks of 4 rows (3-bit, K % 1024 != 0)
    (3, 1024, 50, 6, 64, F32),      # whole-line GEMV once per row (f32 x, 6-bit)
    (6, 512, 96, 4, 64, BF16),      # skinny MFMA GEMV
    (3, 1024, 72, 8, 128, BF16),    # K-split whole-line GEMV (three rows of x, 8-bit)
    (6, 4096, 64, 4, 64, BF16),     # decode MFMA kernel
    (6, 2048, 40, 8, 128, F16),     # mid-M ring kernel (8-bit)
    (32, 2048, 72, 4, 64, BF16),    # small-M GEMM
    (24, 1024, 8300, 3, 64, F16),   # small-M GEMM, two column tiles per block (N > 8192)
    (40, 2560, 200, 4, 64, F16),    # split-K small-M GEMM (10 K parts)
    (96, 512, 136, 4, 64, F16),     # large GEMM
    (3, 96, 20, 4, 32, F32),        # generic kernel (K % 64 != 0)
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: f"M{c[0]}K{c[1]}N{c[2]}b{c[3]}")
@pytest.mark.parametrize("act", [0, 1, 2, 3], ids=["none", "relu", "silu", "gelu"])
def test_fused_bias_activation(ctx, oracle, case, act):
    """op_quantized_matmul_fused: out = act(x . w_hat^T + bias) with the
    bias and activation applied in fp32 by the kernel that computes out,
    against the oracle's fp32 matmul followed by the same stage; f32 output
    at the fp32 gate, plus a bf16-output run at the bf16 gate."""
    from mlx_amd import abi, runtime
    O = oracle
    M, K, N, bits, gs, xd = case
    sbd = F16 if xd == F32 else xd
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=5000 + M + act)
    bias_dt = [F32, F16, BF16, F32][act]
    bias = O.from_f32(O.rng_normal(N, seed=6000 + N), bias_dt)
    gemm = ctx.select_kernel(M, K, N, gs, bits, xd, sbd) == abi.KERNEL_GEMM
    acc = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32,
                             w_round=xd if gemm else F32)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    bb = ctx.upload(bias)
    try:
        for od in (F32, BF16):
            out = ctx.alloc(M * N * runtime.esize(od))
            print(f"[case] fused M={M} K={K} N={N} b={bits} act={act} out={od}", flush=True)
            ctx.quantized_matmul_fused(*bufs, bb, out, M, K, N, gs, bits, xd, sbd, bias_dt, od, act)
            y = out.download(runtime.np_dtype(od), (M, N))
            out.free()
            check_output(O, y, O.fused_epilogue(acc, bias, bias_dt, act, od), od, f"fused act{act} out{od}")
        # no bias: the same as the plain op followed by the activation
        out = ctx.alloc(M * N * 4)
        ctx.quantized_matmul_fused(*bufs, None, out, M, K, N, gs, bits, xd, sbd, F32, F32, act)
        y = out.download(np.float32, (M, N))
        out.free()
        check_output(O, y, O.fused_epilogue(acc, None, F32, act, F32), F32, f"fused act{act} no bias")
    finally:
        for t in bufs + [bb]:
            t.free()


def test_fused_errors(ctx, oracle):
    """Unknown activation, a short bias buffer: INVALID_ARGUMENT; a bias in
    an unsupported dtype: NOT_SUPPORTED; nothing is launched."""
    from mlx_amd import abi, runtime
    O = oracle
    M, K, N = 1, 256, 32
    x, w_q, s, b, _ = O.make_problem(M, K, N, 4, 64, F16, F16, seed=7)
    bufs = [ctx.upload(a) for a in (x, w_q, s, b)]
    out, short, okb = ctx.alloc(M * N * 2), ctx.alloc(N * 2 - 2), ctx.alloc(N * 4)
    try:
        for bias, bdt, act, code in [(okb, F32, 4, abi.ERR_INVALID_ARGUMENT),
                                     (okb, F32, -1, abi.ERR_INVALID_ARGUMENT),
                                     (short, F16, 0, abi.ERR_INVALID_ARGUMENT),
                                     (okb, 7, 0, abi.ERR_NOT_SUPPORTED)]:
            with pytest.raises(runtime.LuxError) as e:
                ctx.quantized_matmul_fused(*bufs, bias, out, M, K, N, 64, 4, F16, F16, bdt, F16, act)
            assert e.value.code == code
    finally:
        for t in bufs + [out, short, okb]:
            t.free()


@pytest.mark.parametrize("M,K,N,bits,gs,xd,sbd,kern", [
    (96, 512, 136, 4, 64, BF16, BF16, "gemm"),   # large GEMM
    (200, 1024, 300, 4, 64, BF16, BF16, "gemm"), # register-W large GEMM
    (130, 2048, 264, 8, 128, F16, F32, "gemm"),  # register-W large GEMM, 8-bit
    (32, 1024, 70, 3, 32, F16, F32, "gemm"),     # small-M GEMM
    (24, 1152, 300, 4, 64, BF16, BF16, "gemm"),  # split-K small-M GEMM (3 K parts)
    (1, 4096, 96, 4, 64, F16, F16, "gemv"),      # whole-line GEMV
    (1, 14336, 40, 4, 64, F16, F16, "gemv"),     # split-K GEMV
    (2, 2048, 48, 8, 64, BF16, BF16, "gemv"),    # K-split whole-line GEMV
    (2, 2048, 48, 3, 64, F16, F16, "gemv"),      # stream GEMV
    (6, 4096, 64, 4, 64, BF16, BF16, "gemv"),    # decode MFMA kernel
    (8, 1024, 40, 8, 128, F16, F16, "gemv"),     # mid-M ring kernel
    (3, 96, 20, 5, 32, F32, F32, "gemv"),        # generic kernel
])
def test_one_hot_rows_select_weight_columns(ctx, oracle, M, K, N, bits, gs, xd, sbd, kern):
    """x row m = e_{k_m} (one 1.0, zeros elsewhere): y[m, :] is column k_m of
    the dequantized weights.  The GEMM kernels round the weights to the
    activation type first, so theirs is round_T(w_hat) bit for bit; the
    GEMV kernels compute the exact form, within the fp32 gate."""
    O = oracle
    _, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=8000 + M)
    ks = np.random.default_rng(M * K).integers(0, K, M)
    xf = np.zeros((M, K), np.float32)
    xf[np.arange(M), ks] = 1.0
    x = O.from_f32(xf, xd)
    y = run(ctx, x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32, KERNELS[kern])
    if kern == "gemm":
        w_t = O.to_f32(O.dequantize(w_q, s, b, K, gs, bits, sbd, xd), xd)
        assert np.array_equal(y.view(np.uint32), np.ascontiguousarray(w_t[:, ks].T).view(np.uint32))
    else:
        w_hat = O.dequantize(w_q, s, b, K, gs, bits, sbd, F32)
        check_output(O, y, np.ascontiguousarray(w_hat[:, ks].T), F32, f"one-hot {kern} M{M}")
    # and x = 0 gives y = 0 on the same path
    y0 = run(ctx, O.from_f32(np.zeros((M, K), np.float32), xd), w_q, s, b, M, K, N, gs, bits, xd, sbd, F32,
             KERNELS[kern])
    assert not np.any(y0)


def test_weights_past_2gib(ctx, oracle):
    """Packed weights larger than 2^31 bytes (K=4096, 4-bit, 1 052 675 rows:
    2 GiB + 8 MB): the GEMV kernels address them with per-block buffer
    bases, the size-limited kernels decline them, and every sampled row --
    the first ones, rows around the 2^31-byte mark, the last block -- equals
    the oracle for M = 1 (whole-line kernel), 3 and 6 (stream kernel, 6 in
    chunks of 4 rows) and 96
    (the large GEMM, whose 32-bit offsets reach 4 GiB)."""
    O = oracle
    K, gs, bits = 4096, 64, 4
    N = (1 << 31) // (K // 2) + 4099
    rng = np.random.default_rng(11)
    w_q = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint32)
    G = K // gs
    s = O.from_f32(rng.uniform(0.001, 0.02, size=(N, G)).astype(np.float32), F16)
    b = O.from_f32(rng.uniform(-0.1, 0.0, size=(N, G)).astype(np.float32), F16)
    mark = (1 << 31) // (K // 2)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(mark - 40, mark + 40),
                                     rng.integers(0, N, 200), np.arange(N - 70, N)]))
    from mlx_amd import abi
    bufs = [ctx.upload(a) for a in (w_q, s, b)]
    try:
        for M in (1, 3, 6, 96):
            x = O.from_f32(O.rng_normal(M * K, 900 + M).reshape(M, K), F16)
            X, Y = ctx.upload(x), ctx.alloc(M * N * 4)
            print(f"[case] qmm M={M} K={K} N={N} (weights {w_q.nbytes} B)", flush=True)
            ctx.quantized_matmul(X, *bufs, Y, M, K, N, gs, bits, F16, F16, F32)
            y = Y.download(np.float32, (M, N))
            X.free()
            Y.free()
            gemm = ctx.select_kernel(M, K, N, gs, bits, F16) == abi.KERNEL_GEMM
            assert gemm == (M > 8)
            want = O.quantized_matmul(x, w_q[rows], s[rows], b[rows], M, K, len(rows), gs, bits, F16, F16, F32,
                                      variant="omp", w_round=F16 if gemm else F32)
            check_output(O, np.ascontiguousarray(y[:, rows]), want, F32, f"2 GiB weights M{M}")
            assert np.all(np.isfinite(y))
    finally:
        for t in bufs:
            t.free()


def test_two_contexts_on_two_threads(oracle):
    """Independent contexts, one caller thread each (the plugin contract):
    both threads run several kernel families at once (ctypes releases the
    GIL around every plugin call) and each result equals the oracle."""
    import threading
    from mlx_amd import runtime
    O = oracle
    cases = [(1, 4096, 2048, 4, 64, F16), (4, 2048, 512, 4, 32, BF16), (32, 2048, 256, 8, 128, BF16),
             (6, 512, 300, 3, 64, F16), (128, 512, 256, 4, 64, F16)]
    problems = [O.make_problem(M, K, N, b, g, xd, xd, seed=9000 + i) for i, (M, K, N, b, g, xd) in enumerate(cases)]
    results, errors = {}, []

    def worker(tid):
        try:
            with runtime.Context(0) as c:
                for rep in range(3):
                    for i, ((M, K, N, b, g, xd), (x, w_q, s, bb, _)) in enumerate(zip(cases, problems)):
                        y = runtime.run_quantized_matmul(c, x, w_q, s, bb, M, K, N, g, b, xd, xd, F32)
                        results[(tid, rep, i)] = y
        except Exception as e:  # reported below, on the main thread
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errors, errors
    assert all(not t.is_alive() for t in ts)
    ctx = runtime.Context(0)
    try:
        for i, ((M, K, N, b, g, xd), (x, w_q, s, bb, _)) in enumerate(zip(cases, problems)):
            gemm = ctx.select_kernel(M, K, N, g, b, xd) == 2
            want = O.quantized_matmul(x, w_q, s, bb, M, K, N, g, b, xd, xd, F32, w_round=xd if gemm else F32)
            for tid in range(2):
                for rep in range(3):
                    check_output(O, results[(tid, rep, i)], want, F32, f"thread {tid} rep {rep} case {i}")
    finally:
        ctx.close()
