"""Pins for the CPU oracle (oracle/lux_cpu_quant.c).

The reference has no quantized matmul and no golden vectors for it, so each
oracle function is pinned by checks that a plausible mistake fails:
  * hand-computed packing known answers, incl. codes straddling words;
  * an independent numpy unpacker (np.unpackbits on the little-endian byte
    stream), and pack/unpack round trips in both directions;
  * f16/bf16 conversions against numpy (f16 exhaustively);
  * dequantization against float64 arithmetic (fmaf = one rounding);
  * quantizer invariants (code range, group min -> 0, error <= scale/2,
    constant groups);
  * matmul against the reference's own 2x2 known answer
    (reference test/test_core.cpp:95-117), against fp64 brute force, against
    exact integer matmul (scale 1, bias 0), and bit for bit against the
    reference CPU backend's op_matmul_f32 (reference src/cpu_backend.cpp:
    243-266, compiled from its source into oracle/_ref) applied to the
    dequantized weights;
  * the dequantize-to-T form (w_round) bit for bit against the same
    reference op on T-rounded weights, and its OpenMP form against fp64.
"""
import ctypes
import hashlib
import os

import numpy as np
import pytest

BITS = [2, 3, 4, 5, 6, 8]


# ---------------------------------------------------------------- packing --

def test_pack_known_answers(oracle):
    O = oracle
    # 4-bit: codes 0..7 -> 0x76543210 (code k at bits 4k..4k+3)
    w = O.pack_bits(np.arange(8, dtype=np.uint8).reshape(1, 8), 4)
    assert w.tolist() == [[0x76543210]]
    # 8-bit: one byte per code, little-endian
    w = O.pack_bits(np.array([[0x11, 0x22, 0x33, 0x44]], dtype=np.uint8), 8)
    assert w.tolist() == [[0x44332211]]
    # 2-bit: 0,1,2,3 repeated -> 0b11100100 per byte
    w = O.pack_bits(np.tile(np.arange(4, dtype=np.uint8), 4).reshape(1, 16), 2)
    assert w.tolist() == [[0xE4E4E4E4]]
    # 3-bit: 32 codes in 3 words; code 0 = 1, code 10 = 7 straddles bits 30..32
    c = np.zeros((1, 32), np.uint8)
    c[0, 0], c[0, 10] = 1, 7
    assert O.pack_bits(c, 3).tolist() == [[0xC0000001, 0x00000001, 0]]
    # 3-bit: code 21 at bits 63..65 straddles words 1 and 2
    c = np.zeros((1, 32), np.uint8)
    c[0, 21] = 5  # 0b101: bit 63 = 1, bits 64..65 = 0b10
    assert O.pack_bits(c, 3).tolist() == [[0, 0x80000000, 0x00000002]]
    # 6-bit: code 5 at bits 30..35
    c = np.zeros((1, 16), np.uint8)
    c[0, 5] = 0x3F
    assert O.pack_bits(c, 6).tolist() == [[0xC0000000, 0x0000000F, 0]]
    # 5-bit: code 6 = 21 = 0b10101 at bits 30..34
    c = np.zeros((1, 32), np.uint8)
    c[0, 6] = 21
    assert O.pack_bits(c, 5).tolist() == [[0x40000000, 0x5, 0, 0, 0]]


def numpy_unpack(w_q, K, bits):
    """Independent unpacker: little-endian bytes -> little-endian bit list."""
    N = w_q.shape[0]
    by = w_q.astype("<u4").view(np.uint8).reshape(N, -1)
    bitsarr = np.unpackbits(by, axis=1, bitorder="little")[:, : K * bits].reshape(N, K, bits)
    return (bitsarr.astype(np.uint32) << np.arange(bits, dtype=np.uint32)).sum(axis=2).astype(np.uint8)


@pytest.mark.parametrize("bits", BITS)
def test_pack_unpack_roundtrips(oracle, bits):
    O = oracle
    rng = np.random.default_rng(bits)
    N, K = 7, 256
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    w = O.pack_bits(codes, bits)
    assert w.shape == (N, K * bits // 32)
    assert np.array_equal(O.unpack_bits(w, K, bits), codes)
    assert np.array_equal(numpy_unpack(w, K, bits), codes)
    # every bit pattern is a valid code stream: unpack then pack is the identity
    words = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(O.pack_bits(O.unpack_bits(words, K, bits), bits), words)
    assert np.array_equal(O.unpack_bits(words, K, bits), numpy_unpack(words, K, bits))


def test_pack_rejects_bad_shapes(oracle):
    O = oracle
    L = O.lib()
    out = np.zeros(4, np.uint32)
    codes = np.zeros(12, np.uint8)
    # K * bits not a multiple of 32
    assert L.lux_cpu_pack_bits(out.ctypes.data, codes.ctypes.data, 1, 12, 3) == 1
    assert L.lux_cpu_pack_bits(out.ctypes.data, codes.ctypes.data, 1, 8, 9) == 1


# ------------------------------------------------------------ conversions --

def test_f16_conversions_match_numpy(oracle):
    O = oracle
    h = np.arange(65536, dtype=np.uint16)
    f = O.to_f32(h, O.F16)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(f.view(np.uint32)[finite], ref.view(np.uint32)[finite])
    assert np.all(np.isnan(f[np.isnan(ref)]))
    xs = [O.rng_normal(1 << 18, 3, 0.0, s) for s in (1e-6, 1e-3, 1.0, 1e3, 4e4)]
    x = np.concatenate(xs + [np.array([65504, 65519.99, 65520, 65536, 2**-24, 2**-25, 3 * 2**-26,
                                       -0.0, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        assert np.array_equal(O.from_f32(x, O.F16), x.astype(np.float16).view(np.uint16))


def test_bf16_conversions(oracle):
    O = oracle
    x = np.concatenate([O.rng_normal(1 << 18, 5, 0.0, s) for s in (1e-30, 1e-3, 1.0, 1e30)])
    b = O.from_f32(x, O.BF16)
    # widening is exact and the rounding is to nearest: no other bf16 is closer
    back = O.to_f32(b, O.BF16).astype(np.float64)
    up = (b.astype(np.uint32) + 1) << 16
    dn = (b.astype(np.uint32) - 1) << 16
    nb_up = up.astype(np.uint32).view(np.float32).astype(np.float64)
    nb_dn = dn.astype(np.uint32).view(np.float32).astype(np.float64)
    err = np.abs(back - x)
    assert np.all(err <= np.abs(nb_up - x)) and np.all(err <= np.abs(nb_dn - x))
    # ties go to the even mantissa
    ties = np.array([0x3F808000, 0x3F818000], np.uint32).view(np.float32)
    assert O.from_f32(ties, O.BF16).tolist() == [0x3F80, 0x3F82]


def test_rng_is_deterministic_and_normal(oracle):
    O = oracle
    a, b = O.rng_normal(1 << 20, 42), O.rng_normal(1 << 20, 42)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, O.rng_normal(1 << 20, 43))
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    assert hashlib.sha256(O.rng_normal(1000, 1).tobytes()).hexdigest() == \
        hashlib.sha256(O.rng_normal(1000, 1).tobytes()).hexdigest()


# ------------------------------------------------------- quantize/dequant --

@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sb", [0, 1, 2])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_invariants(oracle, bits, sb, gs):
    O = oracle
    N, K = 9, 256
    w = O.rng_normal(N * K, 100 + bits, 0.0, 0.02).reshape(N, K)
    w[3, :gs] = 0.125  # a constant group
    w_q, s, b = O.quantize(w, gs, bits, sb)
    q = O.unpack_bits(w_q, K, bits).astype(np.int64)
    assert q.max() <= (1 << bits) - 1
    sf, bf = O.to_f32(s, sb), O.to_f32(b, sb)
    G = K // gs
    # constant group: scale 0, all codes 0, bias = the value
    assert sf[3, 0] == 0 and np.all(q[3, :gs] == 0) and bf[3, 0] == np.float32(0.125)
    wg = w.reshape(N, G, gs)
    qg = q.reshape(N, G, gs)
    mn = wg.min(axis=2)
    # stored scale/bias are the RNE roundings of (max-min)/(2^b-1) and min
    assert np.array_equal(s, O.from_f32((wg.max(axis=2) - mn) / np.float32((1 << bits) - 1), sb))
    assert np.array_equal(b, O.from_f32(mn, sb))
    # reconstruction error per element
    what = O.dequantize(w_q, s, b, K, gs, bits, sb).reshape(N, G, gs).astype(np.float64)
    err = np.abs(what - wg)
    half = 0.5 * sf.astype(np.float64)[..., None]
    if sb == O.F32:
        assert np.all(err <= half * (1 + 1e-5) + 1e-9)
        # the group minimum maps to code 0
        assert np.all(np.take_along_axis(qg, wg.argmin(axis=2)[..., None], 2) == 0)
    else:
        # stored scale/bias are rounded: allow their rounding error over 2^b-1 steps
        ulp = np.float64(2.0 ** (-10 if sb == O.F16 else -7))
        slack = (np.abs(sf.astype(np.float64)) * ulp * ((1 << bits)) +
                 np.abs(bf.astype(np.float64)) * ulp)[..., None]
        assert np.all(err <= half + slack + 1e-9)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("sb", [0, 1, 2])
def test_dequantize_is_single_rounding_fma(oracle, bits, sb):
    O = oracle
    N, K, gs = 5, 128, 64
    w = O.rng_normal(N * K, 7 + bits, 0.0, 0.02).reshape(N, K)
    w_q, s, b = O.quantize(w, gs, bits, sb)
    q = numpy_unpack(w_q, K, bits).astype(np.float64)
    sf = np.repeat(O.to_f32(s, sb).astype(np.float64), gs, axis=1)
    bf = np.repeat(O.to_f32(b, sb).astype(np.float64), gs, axis=1)
    # s*q is exact in float64 and so is the sum here: one rounding to fp32
    expect = (sf * q + bf).astype(np.float32)
    got = O.dequantize(w_q, s, b, K, gs, bits, sb, O.F32)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
    for od in (O.F16, O.BF16):
        assert np.array_equal(O.dequantize(w_q, s, b, K, gs, bits, sb, od), O.from_f32(expect, od))


# ------------------------------------------------------------------ matmul --

def test_reference_2x2_known_answer(oracle):
    """[[1,2],[3,4]] . [[5,6],[7,8]] = [[19,22],[43,50]] (reference
    test/test_core.cpp:95-117): B^T as 4-bit codes with scale 1, bias 0, and
    K padded with zeros to one group of 64."""
    O = oracle
    M, K, N = 2, 64, 2
    x = np.zeros((M, K), np.float32)
    x[:, :2] = [[1, 2], [3, 4]]
    codes = np.zeros((N, K), np.uint8)
    codes[:, :2] = [[5, 7], [6, 8]]
    w_q = O.pack_bits(codes, 4)
    s = np.ones((N, 1), np.float32)
    b = np.zeros((N, 1), np.float32)
    for variant in ("ref", "omp"):
        y = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, 4, O.F32, O.F32, O.F32, variant=variant)
        assert y.tolist() == [[19.0, 22.0], [43.0, 50.0]]


@pytest.mark.parametrize("bits", BITS)
def test_integer_matmul_special_case(oracle, bits):
    """scale 1 and bias 0 reduce the op to an integer matmul, exact in fp32."""
    O = oracle
    rng = np.random.default_rng(bits)
    M, K, N = 3, 128, 17
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    x = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    w_q = O.pack_bits(codes, bits)
    G = K // 64
    s, b = np.ones((N, G), np.float32), np.zeros((N, G), np.float32)
    want = x.astype(np.int64) @ codes.astype(np.int64).T
    for variant in ("ref", "omp"):
        y = O.quantized_matmul(x, w_q, s, b, M, K, N, 64, bits, O.F32, O.F32, O.F32, variant=variant)
        assert np.array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("dt", [(0, 0, 0), (1, 1, 1), (2, 2, 2), (1, 0, 0), (2, 1, 0)])
def test_matmul_matches_fp64_bruteforce(oracle, bits, dt):
    O = oracle
    xd, sbd, od = dt
    for M, K, N, gs in [(1, 64, 5, 64), (3, 128, 33, 32), (5, 256, 8, 128)]:
        x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=bits * 7 + M)
        what = O.dequantize(w_q, s, b, K, gs, bits, sbd).astype(np.float64)
        xf = O.to_f32(x, xd).astype(np.float64)
        exact = xf @ what.T
        y64 = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od, variant="f64")
        assert np.allclose(y64, exact, rtol=1e-12, atol=1e-12)
        scale = np.abs(exact).max()
        for variant in ("ref", "omp"):
            y = O.to_f32(O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, od,
                                            variant=variant), od).astype(np.float64)
            # output rounding (f16/bf16) plus fp32 accumulation
            tol = {0: 1e-5, 1: 1e-3, 2: 8e-3}[od]
            assert np.abs(y - exact).max() <= tol * scale


def test_zero_input_gives_zero(oracle):
    O = oracle
    x, w_q, s, b, _ = O.make_problem(2, 128, 9, 4, 64, O.F16, O.F16, seed=3)
    x[:] = 0
    y = O.quantized_matmul(x, w_q, s, b, 2, 128, 9, 64, 4, O.F16, O.F16, O.F16)
    assert np.all(O.to_f32(y, O.F16) == 0)


def _ref_cpu_backend():
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "oracle", "_ref", "libref_cpu_backend.so")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (reference sources absent when it was built)")
    from mlx_amd import abi
    lib = ctypes.CDLL(path)
    desc = abi.BackendDesc()
    init = abi.INIT_FN(("cpu_backend_init", lib))
    assert init(ctypes.byref(desc)) and desc.abi_version == abi.ABI_VERSION
    return lib, desc


def ref_dense_matmul(desc, a, bmat):
    """C = A.B through the reference CPU backend's vtable (op_matmul_f32)."""
    vt = desc.vtbl.contents
    M, K = a.shape
    N = bmat.shape[1]
    ctx = vt.create_context(0)
    ba = vt.buffer_alloc_with_data(ctx, a.ctypes.data, a.nbytes)
    bb = vt.buffer_alloc_with_data(ctx, bmat.ctypes.data, bmat.nbytes)
    bc = vt.buffer_alloc(ctx, M * N * 4)
    assert vt.op_matmul_f32(ctx, ba, bb, bc, M, K, N) == 0
    c = np.empty((M, N), np.float32)
    assert vt.buffer_copy_to_host(ctx, bc, c.ctypes.data, c.nbytes) == 0
    for h in (ba, bb, bc):
        vt.buffer_free(ctx, h)
    vt.destroy_context(ctx)
    return c


@pytest.mark.parametrize("bits", [3, 4, 8])
def test_bit_exact_vs_reference_cpu_backend(oracle, bits):
    """The oracle equals "dequantize on the host, then the reference CPU
    backend's op_matmul_f32" bit for bit: both accumulate fp32 products in
    ascending k with a separate multiply and add."""
    O = oracle
    _, desc = _ref_cpu_backend()
    M, K, N, gs = 4, 512, 40, 64
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, O.F32, O.F32, seed=11)
    what = O.dequantize(w_q, s, b, K, gs, bits, O.F32)
    c = ref_dense_matmul(desc, np.ascontiguousarray(x), np.ascontiguousarray(what.T))
    y = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, O.F32, O.F32, O.F32)
    assert np.array_equal(y.view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("bits", [3, 4, 8])
@pytest.mark.parametrize("wt", [1, 2])
def test_wround_bit_exact_vs_reference_cpu_backend(oracle, bits, wt):
    """The dequantize-to-T form (the GEMM's semantics) equals the reference
    CPU backend's op_matmul_f32 applied to the dequantized weights rounded to
    T (f16 / bf16) and widened back, bit for bit; the OpenMP form of it stays
    within fp32 accumulation error of the fp64 product of the same operands."""
    O = oracle
    _, desc = _ref_cpu_backend()
    M, K, N, gs = 5, 512, 36, 64
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, wt, wt, seed=13 + bits)
    what_t = O.to_f32(O.dequantize(w_q, s, b, K, gs, bits, wt, out_dtype=wt), wt)
    # the rounding is visible: the T-rounded weights differ from the fp32 ones
    assert not np.array_equal(what_t, O.dequantize(w_q, s, b, K, gs, bits, wt))
    xf = np.ascontiguousarray(O.to_f32(x, wt))
    c = ref_dense_matmul(desc, xf, np.ascontiguousarray(what_t.T))
    y = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, wt, wt, O.F32, w_round=wt)
    assert np.array_equal(y.view(np.uint32), c.view(np.uint32))
    exact = xf.astype(np.float64) @ what_t.astype(np.float64).T
    yo = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, wt, wt, O.F32, variant="omp",
                            threads=2, w_round=wt)
    assert np.abs(yo - exact).max() <= 1e-5 * np.abs(exact).max()


def test_check_args(oracle):
    O = oracle
    assert O.check_args(1, 4096, 4096, 64, 4, 0, 0, 0) == 0
    assert O.check_args(1, 4096, 4096, 64, 7, 0, 0, 0) == 3     # bits
    assert O.check_args(1, 4096, 4096, 48, 4, 0, 0, 0) == 3     # group size
    assert O.check_args(1, 4000, 4096, 64, 4, 0, 0, 0) == 1     # K % group
    assert O.check_args(1, 4096, 4096, 64, 4, 4, 0, 0) == 3     # dtype
    assert O.check_args(-1, 4096, 4096, 64, 4, 0, 0, 0) == 1


# ------------------------------------------------------ fused output stage --

def test_activation_closed_forms(oracle):
    """The fused op's activations: exact identities and known values that a
    dropped term, a wrong sign or a wrong constant fails."""
    O = oracle
    v = np.linspace(-8.0, 8.0, 4001)
    for act in (O.ACT_SILU, O.ACT_GELU):
        # f(v) - f(-v) = v for both (f(v) = v * c(v) with c(v) + c(-v) = 1)
        assert np.allclose(O.activation(v, act) - O.activation(-v, act), v, rtol=0, atol=1e-12)
        assert O.activation(np.array([0.0]), act)[0] == 0.0
    # known values: silu(1) = 1 / (1 + e^-1), gelu(1) = Phi(1), gelu(-1) = -(1 - Phi(1))
    assert abs(O.activation(np.array([1.0]), O.ACT_SILU)[0] - 0.7310585786300049) < 1e-15
    assert abs(O.activation(np.array([1.0]), O.ACT_GELU)[0] - 0.8413447460685429) < 1e-15
    assert abs(O.activation(np.array([-1.0]), O.ACT_GELU)[0] + 0.15865525393145707) < 1e-15
    # large |v|: silu and gelu approach relu
    big = np.array([-40.0, 40.0])
    for act in (O.ACT_SILU, O.ACT_GELU):
        assert np.allclose(O.activation(big, act), [0.0, 40.0], atol=1e-12)
    r = O.activation(np.array([-2.0, -0.0, 0.0, 3.5, np.nan]), O.ACT_RELU)
    assert r[0] == 0 and r[3] == 3.5 and np.isnan(r[4])
    assert np.array_equal(O.activation(v, O.ACT_NONE), v)


def test_fused_epilogue_bias_and_rounding(oracle):
    """bias is added in fp32 per column; the result is rounded once to
    fp32 and then to the output type."""
    O = oracle
    acc = np.array([[1.0, -2.0, 0.5], [3.0, 0.25, -7.0]], np.float32)
    bias = O.from_f32(np.array([0.5, 1.0, -0.5], np.float32), O.F16)
    got = O.fused_epilogue(acc, bias, O.F16, O.ACT_RELU, O.F32)
    assert np.array_equal(got, np.array([[1.5, 0.0, 0.0], [3.5, 1.25, 0.0]], np.float32))
    got = O.fused_epilogue(acc, None, O.F32, O.ACT_NONE, O.BF16)
    assert np.array_equal(O.to_f32(got, O.BF16), acc)
    # fp32 addition, not float64: 1 + 2^-30 rounds to 1
    one = np.array([[1.0]], np.float32)
    tiny = np.array([2.0 ** -30], np.float32)
    assert O.fused_epilogue(one, tiny, O.F32, O.ACT_NONE, O.F32)[0, 0] == np.float32(1.0)
