"""The core-side library (include/lux_quant_core.h), on the CPU: backend
selection the reference loader's way plus LUX_BACKEND and the "hip" name
(reference src/plugin_loader.hpp:112-262), its failure paths, and the
public lux_tensor_quantized_matmul end to end through a fake plugin that
implements the quantized table on the host (tests/fake_plugins).  The
same op on the real plugin and GPU is in test_gpu_core_shim.py."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE_SRC = os.path.join(ROOT, "tests", "fake_plugins", "fake_plugin.c")
F32, F16, BF16, U32 = 0, 1, 2, 100
INVALID, NOT_SUPPORTED = 1, 3


def core_lib():
    """ctypes view of libluxgpu_quant_core.so (a fresh handle per call keeps
    nothing cached between tests; the library itself holds no state)."""
    import mlx_amd
    assert os.path.exists(mlx_amd.CORE_PATH), "run __graft_entry__.build() first"
    L = ctypes.CDLL(mlx_amd.CORE_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    P, I, I64, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.lux_qcore_open.restype = P
    L.lux_qcore_open.argtypes = [ctypes.c_char_p, I, ctypes.POINTER(ctypes.c_char_p)]
    L.lux_qcore_close.argtypes = [P]
    L.lux_qcore_backend_name.restype = ctypes.c_char_p
    L.lux_qcore_backend_name.argtypes = [P]
    for f in ("lux_qcore_vtbl", "lux_qcore_quant", "lux_qcore_context"):
        getattr(L, f).restype = P
        getattr(L, f).argtypes = [P]
    L.lux_qtensor_create.restype = P
    L.lux_qtensor_create.argtypes = [P, P, I64, I64, I]
    L.lux_qtensor_to_host.restype = I
    L.lux_qtensor_to_host.argtypes = [P, P, P, S]
    L.lux_qtensor_free.argtypes = [P, P]
    L.lux_qtensor_dim.restype = I64
    L.lux_qtensor_dim.argtypes = [P, I]
    L.lux_qtensor_dtype.restype = I
    L.lux_qtensor_dtype.argtypes = [P]
    L.lux_tensor_quantized_matmul.restype = P
    L.lux_tensor_quantized_matmul.argtypes = [P, P, P, P, P, I, I, ctypes.POINTER(I)]
    return L


def open_core(L, name=None):
    err = ctypes.c_char_p()
    c = L.lux_qcore_open(name.encode() if name else None, 0, ctypes.byref(err))
    return c, (err.value.decode() if err.value else None)


def fake(tmp_path, name, *defs, subdir="p"):
    d = tmp_path / subdir
    d.mkdir(exist_ok=True)
    so = d / f"libluxgpu_backend_{name}.so"
    r = subprocess.run(["gcc", "-std=c11", "-shared", "-fPIC", f'-DFAKE_NAME="{name}"', *defs, FAKE_SRC,
                        "-lm", "-o", str(so)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return d


@pytest.fixture
def env(monkeypatch):
    """A clean selection environment: only the paths a test sets."""
    monkeypatch.delenv("LUX_BACKEND", raising=False)
    monkeypatch.delenv("LUX_GPU_BACKEND_PATH", raising=False)
    return monkeypatch


def test_explicit_and_priority_selection(tmp_path, env):
    L = core_lib()
    d = fake(tmp_path, "webgpu", "-DFAKE_QUANT")
    fake(tmp_path, "hip", "-DFAKE_QUANT")
    env.setenv("LUX_GPU_BACKEND_PATH", str(d))
    c, err = open_core(L)                      # auto: hip ranks ahead of webgpu
    assert c and err is None and L.lux_qcore_backend_name(c) == b"hip"
    assert L.lux_qcore_vtbl(c) and L.lux_qcore_quant(c) and L.lux_qcore_context(c)
    L.lux_qcore_close(c)
    fake(tmp_path, "metal", "-DFAKE_QUANT")
    c, _ = open_core(L)                        # metal ranks first
    assert L.lux_qcore_backend_name(c) == b"metal"
    L.lux_qcore_close(c)
    env.setenv("LUX_BACKEND", "WebGPU")        # explicit, case-insensitive
    c, _ = open_core(L)
    assert L.lux_qcore_backend_name(c) == b"webgpu"
    L.lux_qcore_close(c)
    c, _ = open_core(L, "hip")                 # an argument wins over LUX_BACKEND
    assert L.lux_qcore_backend_name(c) == b"hip"
    L.lux_qcore_close(c)


def test_search_path_order(tmp_path, env):
    """Each LUX_GPU_BACKEND_PATH entry goes in front, so the last one is
    searched first (reference src/plugin_loader.hpp:135-141)."""
    L = core_lib()
    a = fake(tmp_path, "cuda", "-DFAKE_QUANT", subdir="a")
    b = fake(tmp_path, "cuda", "-DFAKE_QUANT", "-DFAKE_NULL_CTX", subdir="b")
    env.setenv("LUX_GPU_BACKEND_PATH", f"{a}:{b}")
    assert open_core(L, "cuda") == (None, "create_context failed")   # b first
    env.setenv("LUX_GPU_BACKEND_PATH", f"{b}:{a}")
    c, _ = open_core(L, "cuda")
    assert c
    L.lux_qcore_close(c)


def test_failure_paths(tmp_path, env, capfd):
    L = core_lib()
    d = fake(tmp_path, "metal")                                  # no quantized table
    fake(tmp_path, "cuda", "-DFAKE_QUANT", "-DFAKE_INIT_FALSE")  # no device
    fake(tmp_path, "webgpu", "-DFAKE_QUANT", "-DFAKE_ABI=1")     # old ABI
    env.setenv("LUX_GPU_BACKEND_PATH", str(d))
    assert open_core(L, "metal") == (None, "backend has no quantized-matmul extension")
    assert open_core(L, "cuda") == (None, "backend unavailable")
    assert open_core(L, "webgpu") == (None, "ABI version mismatch")
    assert "has ABI version 1, expected 2" in capfd.readouterr().err
    assert open_core(L, "vulkan") == (None, "backend not found")
    c, err = open_core(L)
    if c:  # a GPU machine: the real plugin next to the library is available
        assert L.lux_qcore_backend_name(c) == b"hip"
        L.lux_qcore_close(c)
    else:
        assert err == "no backend available"
    env.setenv("LUX_BACKEND", "cpu")
    c, err = open_core(L)
    assert c is None and "CPU backend" in err


def test_quantized_matmul_through_a_fake_backend(tmp_path, env, oracle):
    """Shapes, output allocation and the call through the plugin table,
    against the oracle (f32, the fake's only dtypes)."""
    L = core_lib()
    env.setenv("LUX_GPU_BACKEND_PATH", str(fake(tmp_path, "metal", "-DFAKE_QUANT")))
    c, _ = open_core(L)
    M, K, N, gs, bits = 3, 256, 20, 64, 3
    x, w_q, s, b, _ = oracle.make_problem(M, K, N, bits, gs, F32, F32, seed=3)
    T = lambda a, dt: L.lux_qtensor_create(c, a.ctypes.data, a.shape[0], a.shape[1], dt)
    X, W, S, B = T(x, F32), T(w_q, U32), T(s, F32), T(b, F32)
    assert (L.lux_qtensor_dim(W, 0), L.lux_qtensor_dim(W, 1), L.lux_qtensor_dtype(W)) == (N, K * bits // 32, U32)
    code = ctypes.c_int(-1)
    Y = L.lux_tensor_quantized_matmul(c, X, W, S, B, gs, bits, ctypes.byref(code))
    assert Y and code.value == 0
    assert (L.lux_qtensor_dim(Y, 0), L.lux_qtensor_dim(Y, 1), L.lux_qtensor_dtype(Y)) == (M, N, F32)
    y = np.empty((M, N), np.float32)
    assert L.lux_qtensor_to_host(c, Y, y.ctypes.data, y.nbytes) == 0
    want = oracle.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, F32, F32, F32)
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    # shape and dtype mismatches: NULL, INVALID_ARGUMENT, nothing launched
    S2 = L.lux_qtensor_create(c, None, N, K // gs, F16)
    W2 = L.lux_qtensor_create(c, None, N, K * bits // 32, F32)
    for args in [(X, W, S, B, gs, 4), (X, W, S, B, 32, bits), (X, W, S2, B, gs, bits), (X, W2, S, B, gs, bits),
                 (W, W, S, B, gs, bits), (X, W, S, None, gs, bits)]:
        code.value = -1
        assert not L.lux_tensor_quantized_matmul(c, *args, ctypes.byref(code))
        assert code.value == INVALID
    # the backend's own error comes back (the fake runs f32 only)
    X16 = L.lux_qtensor_create(c, None, M, K, F16)
    assert not L.lux_tensor_quantized_matmul(c, X16, W, S, B, gs, bits, ctypes.byref(code))
    assert code.value == NOT_SUPPORTED
    # zero-filled creation, and bad shapes or dtypes are refused
    Z = L.lux_qtensor_create(c, None, 2, 3, F32)
    z = np.ones((2, 3), np.float32)
    L.lux_qtensor_to_host(c, Z, z.ctypes.data, z.nbytes)
    assert not z.any()
    assert not L.lux_qtensor_create(c, None, -1, 3, F32) and not L.lux_qtensor_create(c, None, 2, 3, 7)
    for t in (X, W, S, B, Y, S2, W2, X16, Z):
        L.lux_qtensor_free(c, t)
    L.lux_qcore_close(c)


def test_real_plugin_without_gpu_is_unavailable(env):
    if os.path.exists("/dev/kfd"):
        pytest.skip("a ROCm device node is present")
    L = core_lib()
    assert open_core(L, "hip") == (None, "backend unavailable")
