"""bench.py's synthetic inputs are the test fixtures' tensors: its generator
(in the bench support library, libluxgpu_ceiling.so) draws the same streams
as the oracle's, and the c0 and c4 inputs it builds quantize to the
committed digests."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

F32, F16 = 0, 1


@pytest.fixture(scope="module")
def bench():
    import bench as b
    if not os.path.exists(os.path.join(ROOT, "mlx_amd", "lib", "libluxgpu_ceiling.so")):
        pytest.skip("bench support library not built")
    return b


def test_generator_streams_equal_the_oracle(bench, oracle):
    for n, seed, std in ((1, 3, 1.0), (1001, 5, 1.0), (65536, 6, 0.02)):
        assert np.array_equal(bench.rng_normal(n, seed, std).view(np.uint32),
                              oracle.rng_normal(n, seed, 0.0, std).view(np.uint32)), (n, seed)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("name,M,K,N,bits,gs,xd,outliers", [
    ("c0", 1, 4096, 4096, 4, 64, F32, False),
    ("c4_b3", 64, 4096, 11008, 3, 64, F16, True),
])
def test_inputs_hash_to_the_committed_digests(bench, oracle, name, M, K, N, bits, gs, xd, outliers):
    with open(os.path.join(ROOT, "tests", "golden", "digests.json")) as f:
        want = json.load(f)[name]
    x = bench.x_host(M, K, xd, 1)
    w = bench.w_host(N, K, 1, outliers)
    w_q, s, b = oracle.quantize(np.array(w), gs, bits, xd)
    got = {"x": _sha(x), "w_q": _sha(w_q), "scales": _sha(s), "biases": _sha(b)}
    assert got == want["sha256"]
    assert bench.digest_match(K, N, bits, gs, xd, 1, outliers, w_q, s, b) is True
    assert bench.digest_match(K, N, bits, gs, xd, 2, outliers, w_q, s, b) is None
