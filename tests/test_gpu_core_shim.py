"""lux_tensor_quantized_matmul through the core-side library on the real
plugin: automatic selection finds "hip" next to the library, and the op
matches the oracle at c1 (M = 1 and 8) and on a GEMM shape."""
import ctypes

import numpy as np
import pytest

from qmm_util import BF16, F16, F32, check_output
from test_core_shim import U32, core_lib, open_core

pytestmark = pytest.mark.gpu


def test_core_library_runs_the_plugin(oracle, monkeypatch):
    monkeypatch.delenv("LUX_BACKEND", raising=False)
    monkeypatch.delenv("LUX_GPU_BACKEND_PATH", raising=False)
    L = core_lib()
    c, err = open_core(L)
    assert c, err
    assert L.lux_qcore_backend_name(c) == b"hip"
    try:
        for (M, K, N, gs, bits, xd) in [(1, 4096, 14336, 64, 4, F16), (8, 4096, 14336, 64, 4, F16),
                                        (96, 1024, 320, 64, 4, BF16)]:
            print(f"[case] core M={M} K={K} N={N}", flush=True)
            x, w_q, s, b, _ = oracle.make_problem(M, K, N, bits, gs, xd, xd, seed=17 + M)
            ts = [L.lux_qtensor_create(c, a.ctypes.data, a.shape[0], a.shape[1], dt)
                  for a, dt in ((x, xd), (w_q, U32), (s, xd), (b, xd))]
            code = ctypes.c_int(-1)
            Y = L.lux_tensor_quantized_matmul(c, *ts, gs, bits, ctypes.byref(code))
            assert Y and code.value == 0
            y = np.empty((M, N), np.uint16)
            assert L.lux_qtensor_to_host(c, Y, y.ctypes.data, y.nbytes) == 0
            q = L.lux_qcore_quant(c)
            from mlx_amd import abi
            qt = ctypes.cast(q, ctypes.POINTER(abi.QuantVtbl)).contents
            gemm = qt.select_kernel(M, K, N, gs, bits, xd, xd) == abi.KERNEL_GEMM
            want = oracle.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, xd, xd, variant="omp",
                                           w_round=xd if gemm else F32)
            check_output(oracle, y, want, xd, f"core M{M}")
            for t in ts + [Y]:
                L.lux_qtensor_free(c, t)
    finally:
        L.lux_qcore_close(c)
