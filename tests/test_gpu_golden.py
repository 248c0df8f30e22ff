"""The HIP plugin against the committed golden fixtures directly (no oracle
run): quantize bit for bit, dequantize bit for bit, the GEMV within the fp32
gate (rows whose weights are all finite; rows holding inf or NaN weights
must come out non-finite)."""
import os

import numpy as np
import pytest

from qmm_util import F32, rel_err

HERE = os.path.dirname(os.path.abspath(__file__))


def load():
    z = np.load(os.path.join(HERE, "golden", "golden.npz"))
    keys = sorted({k.split("/")[0] for k in z.files})
    return {k: {n.split("/")[1]: z[n] for n in z.files if n.startswith(k + "/")} for k in keys}


CASES = load()


def bits_of(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint16)


@pytest.mark.gpu
@pytest.mark.parametrize("key", sorted(CASES))
def test_plugin_matches_golden(ctx, key):
    from mlx_amd import abi, runtime
    c = CASES[key]
    M, K, N, bits, gs, xd, sbd = (int(v) for v in c["meta"])
    print(f"[case] golden {key}", flush=True)
    w_q, s, b = runtime.run_quantize(ctx, c["w"], gs, bits, F32, sbd)
    assert np.array_equal(w_q, c["w_q"])
    assert np.array_equal(bits_of(s), bits_of(c["s"])) and np.array_equal(bits_of(b), bits_of(c["b"]))
    deq = runtime.run_dequantize(ctx, c["w_q"], c["s"], c["b"], K, gs, bits, sbd, F32)
    assert np.array_equal(bits_of(deq), bits_of(c["deq"]))
    y = runtime.run_quantized_matmul(ctx, c["x"], c["w_q"], c["s"], c["b"], M, K, N, gs, bits, xd, sbd, F32,
                                     abi.KERNEL_GEMV)
    rows = np.all(np.isfinite(c["deq"]), axis=1)
    assert rel_err(y[:, rows], c["y"][:, rows]) <= 1e-5
    assert not np.isfinite(y[:, ~rows]).any()
