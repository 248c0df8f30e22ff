"""numpy front end of the CPU oracle (oracle/liblux_cpu_quant.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the mlx_amd package.

Every function returns numpy arrays; 16-bit floats travel as uint16 bit
patterns (numpy has no bfloat16).  Dtype codes are LuxBackendDtype
(reference include/lux/gpu/backend_plugin.h:38-47): 0 f32, 1 f16, 2 bf16.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblux_cpu_quant.so")
REF_CPU_BACKEND = os.path.join(HERE, "_ref", "libref_cpu_backend.so")

F32, F16, BF16 = 0, 1, 2
_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16}

_lib = None


def build() -> None:
    """Compile the oracle (and, where the reference is mounted, _ref/)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, U64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_size_t
        L.lux_cpu_f32_to_f16.argtypes = [ctypes.c_float]
        L.lux_cpu_f32_to_f16.restype = ctypes.c_uint16
        L.lux_cpu_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.lux_cpu_f16_to_f32.restype = ctypes.c_float
        L.lux_cpu_f32_to_bf16.argtypes = [ctypes.c_float]
        L.lux_cpu_f32_to_bf16.restype = ctypes.c_uint16
        L.lux_cpu_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.lux_cpu_bf16_to_f32.restype = ctypes.c_float
        L.lux_cpu_convert.argtypes = [P, I, P, I, SZ]
        L.lux_cpu_convert.restype = None
        L.lux_cpu_rng_normal_f32.argtypes = [P, SZ, U64, ctypes.c_float, ctypes.c_float]
        L.lux_cpu_rng_normal_f32.restype = None
        L.lux_cpu_rng_u32.argtypes = [P, SZ, U64]
        L.lux_cpu_rng_u32.restype = None
        L.lux_cpu_pack_bits.argtypes = [P, P, I, I, I]
        L.lux_cpu_unpack_bits.argtypes = [P, P, I, I, I]
        L.lux_cpu_quantize.argtypes = [P, P, P, P, I, I, I, I, I]
        L.lux_cpu_dequantize.argtypes = [P, P, P, P, I, I, I, I, I, I]
        L.lux_cpu_quantized_matmul.argtypes = [P, P, P, P, P] + [I] * 8
        L.lux_cpu_quantized_matmul_f64.argtypes = [P, P, P, P, P] + [I] * 7
        L.lux_cpu_quantized_matmul_omp.argtypes = [P, P, P, P, P] + [I] * 9
        L.lux_cpu_quantized_matmul_wround.argtypes = [P, P, P, P, P] + [I] * 9
        L.lux_cpu_quantized_matmul_wround_omp.argtypes = [P, P, P, P, P] + [I] * 10
        L.lux_cpu_quant_check.argtypes = [I] * 8
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"{what} failed with LuxBackendError {rc}")


# ---- conversions -----------------------------------------------------------

def convert(a: np.ndarray, in_dtype: int, out_dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=_NP[in_dtype])
    out = np.empty(a.shape, dtype=_NP[out_dtype])
    lib().lux_cpu_convert(_p(out), out_dtype, _p(a), in_dtype, a.size)
    return out


def to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    return convert(a, dtype, F32)


def from_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    return convert(np.asarray(a, dtype=np.float32), F32, dtype)


# ---- PRNG ------------------------------------------------------------------

def rng_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().lux_cpu_rng_normal_f32(_p(out), n, seed, mean, std)
    return out


def rng_u32(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().lux_cpu_rng_u32(_p(out), n, seed)
    return out


# ---- format ----------------------------------------------------------------

def pack_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    N, K = codes.shape
    out = np.empty((N, K * bits // 32), dtype=np.uint32)
    _check(lib().lux_cpu_pack_bits(_p(out), _p(codes), N, K, bits), "pack_bits")
    return out


def unpack_bits(w_q: np.ndarray, K: int, bits: int) -> np.ndarray:
    w_q = np.ascontiguousarray(w_q, dtype=np.uint32)
    N = w_q.shape[0]
    out = np.empty((N, K), dtype=np.uint8)
    _check(lib().lux_cpu_unpack_bits(_p(out), _p(w_q), N, K, bits), "unpack_bits")
    return out


def quantize(w: np.ndarray, group_size: int, bits: int, sb_dtype: int):
    """fp32 W[N, K] -> (w_q uint32[N, K*bits/32], scales, biases [N, K/g])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    w_q = np.empty((N, K * bits // 32), dtype=np.uint32)
    s = np.empty((N, K // group_size), dtype=_NP[sb_dtype])
    b = np.empty((N, K // group_size), dtype=_NP[sb_dtype])
    _check(lib().lux_cpu_quantize(_p(w_q), _p(s), _p(b), _p(w), N, K, group_size, bits, sb_dtype),
           "quantize")
    return w_q, s, b


def dequantize(w_q, scales, biases, K: int, group_size: int, bits: int,
               sb_dtype: int, out_dtype: int = F32) -> np.ndarray:
    N = w_q.shape[0]
    out = np.empty((N, K), dtype=_NP[out_dtype])
    args = [np.ascontiguousarray(a) for a in (w_q, scales, biases)]
    _check(lib().lux_cpu_dequantize(_p(out), *[_p(a) for a in args], N, K, group_size,
                                    bits, sb_dtype, out_dtype), "dequantize")
    return out


def quantized_matmul(x, w_q, scales, biases, M: int, K: int, N: int, group_size: int,
                     bits: int, x_dtype: int, sb_dtype: int, out_dtype: int,
                     variant: str = "ref", threads: int = 0, w_round: int = F32) -> np.ndarray:
    """y[M, N] = x[M, K] . dequant(W)[N, K]^T.

    variant "ref": scalar oracle;  "f64": fp64 accumulation (returns float64);
    "omp": the timed OpenMP baseline.
    w_round F16/BF16: the dequantized weight is rounded to that type before
    the multiply (the GEMM's "dequantize to the activation type" semantics);
    with variant "ref" the scalar oracle, with "omp" its OpenMP form.
    """
    args = [np.ascontiguousarray(a) for a in (x, w_q, scales, biases)]
    L = lib()
    if variant == "f64":
        y = np.empty((M, N), dtype=np.float64)
        _check(L.lux_cpu_quantized_matmul_f64(_p(y), *[_p(a) for a in args], M, K, N,
                                              group_size, bits, x_dtype, sb_dtype), "matmul_f64")
        return y
    y = np.empty((M, N), dtype=_NP[out_dtype])
    if w_round != F32:
        if variant == "ref":
            rc = L.lux_cpu_quantized_matmul_wround(_p(y), *[_p(a) for a in args], M, K, N, group_size,
                                                   bits, x_dtype, sb_dtype, out_dtype, w_round)
        elif variant == "omp":
            rc = L.lux_cpu_quantized_matmul_wround_omp(_p(y), *[_p(a) for a in args], M, K, N,
                                                       group_size, bits, x_dtype, sb_dtype, out_dtype,
                                                       w_round, threads)
        else:
            raise ValueError(variant)
        _check(rc, "quantized_matmul_wround")
        return y
    if variant == "ref":
        rc = L.lux_cpu_quantized_matmul(_p(y), *[_p(a) for a in args], M, K, N, group_size,
                                        bits, x_dtype, sb_dtype, out_dtype)
    elif variant == "omp":
        rc = L.lux_cpu_quantized_matmul_omp(_p(y), *[_p(a) for a in args], M, K, N, group_size,
                                            bits, x_dtype, sb_dtype, out_dtype, threads)
    else:
        raise ValueError(variant)
    _check(rc, "quantized_matmul")
    return y


ACT_NONE, ACT_RELU, ACT_SILU, ACT_GELU = 0, 1, 2, 3


def _erf(v: np.ndarray) -> np.ndarray:
    from scipy.special import erf
    return erf(v)


def activation(v: np.ndarray, act: int) -> np.ndarray:
    """The fused op's activations in float64 (no reference counterpart; the
    plugin header lux_gpu_quant_backend.h defines them):
    relu(v) = v < 0 ? 0 : v (NaN passes), silu(v) = v / (1 + exp(-v)),
    gelu(v) = v/2 (1 + erf(v / sqrt 2))."""
    v = np.asarray(v, np.float64)
    if act == ACT_NONE:
        return v
    if act == ACT_RELU:
        return np.where(v < 0, 0.0, v)
    if act == ACT_SILU:
        with np.errstate(over="ignore"):
            return v / (1.0 + np.exp(-v))
    if act == ACT_GELU:
        return 0.5 * v * (1.0 + _erf(v / np.sqrt(2.0)))
    raise ValueError(act)


def fused_epilogue(acc: np.ndarray, bias, bias_dtype: int, act: int, out_dtype: int) -> np.ndarray:
    """out = round_out(act(acc + bias[n])) for an fp32 accumulator [M, N]
    (the oracle's quantized_matmul with out_dtype FLOAT32): the bias add in
    fp32 as the kernels do it, the activation in float64, one rounding to
    fp32 and then to out_dtype."""
    v = np.asarray(acc, np.float32)
    if bias is not None:
        v = (v + to_f32(np.asarray(bias), bias_dtype)[None, :]).astype(np.float32)
    return from_f32(activation(v, act).astype(np.float32), out_dtype)


def check_args(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype) -> int:
    return lib().lux_cpu_quant_check(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype)


# ---- synthetic problem generation -----------------

def make_problem(M: int, K: int, N: int, bits: int, group_size: int, x_dtype: int,
                 sb_dtype: int, seed: int, w_std: float = 0.02, outlier_frac: float = 0.0,
                 outlier_scale: float = 20.0):
    """Seeded inputs as the configs describe: x ~ N(0,1) cast to x_dtype,
    W ~ N(0, w_std) (optionally with an exact fraction of entries scaled by
    outlier_scale, chosen by a seeded shuffle), quantized by the oracle."""
    x32 = rng_normal(M * K, seed * 4 + 1).reshape(M, K)
    w = rng_normal(N * K, seed * 4 + 2, 0.0, w_std).reshape(N, K)
    if outlier_frac > 0:
        n_out = int(round(outlier_frac * N * K))
        perm = rng_u32(N * K, seed * 4 + 3).argsort(kind="stable")[:n_out]
        w.reshape(-1)[perm] *= np.float32(outlier_scale)
    x = from_f32(x32, x_dtype)
    w_q, s, b = quantize(w, group_size, bits, sb_dtype)
    return x, w_q, s, b, w
