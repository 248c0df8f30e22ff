"""The committed golden fixtures (tests/golden/, written by
tests/golden/make_fixtures.py) against the CPU oracle and against
restatements that share no code with it:

* the oracle reproduces every fixture bit for bit (quantize, dequantize,
  matmul) -- any change to its conventions shows here;
* the fixtures' packed codes, unpacked with numpy's bit unpacking of the
  little-endian byte stream, give back codes whose fmaf(s, q, b) (exact in
  float64, one rounding to float32) is the fixture's dequantized weight;
* the fixture's y is the float64 product x . deq^T within fp32 accumulation
  error (1e-5 of max|y|);
* the full-size synthetic tensors of every BASELINE config hash to the
  committed digests (generator and quantizer at full size)."""
import hashlib
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
F32, F16, BF16 = 0, 1, 2


def cases():
    z = np.load(os.path.join(GOLD, "golden.npz"))  # allow_pickle defaults to False
    keys = sorted({k.split("/")[0] for k in z.files})
    return {k: {n.split("/")[1]: z[n] for n in z.files if n.startswith(k + "/")} for k in keys}


CASES = cases()


def bits_of(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint16)


@pytest.mark.parametrize("key", sorted(CASES))
def test_oracle_reproduces_fixture(oracle, key):
    O = oracle
    c = CASES[key]
    M, K, N, bits, gs, xd, sbd = (int(v) for v in c["meta"])
    w_q, s, b = O.quantize(c["w"], gs, bits, sbd)
    assert np.array_equal(w_q, c["w_q"])
    assert np.array_equal(bits_of(s), bits_of(c["s"])) and np.array_equal(bits_of(b), bits_of(c["b"]))
    deq = O.dequantize(c["w_q"], c["s"], c["b"], K, gs, bits, sbd)
    assert np.array_equal(bits_of(deq), bits_of(c["deq"]))
    y = O.quantized_matmul(c["x"], c["w_q"], c["s"], c["b"], M, K, N, gs, bits, xd, sbd, F32)
    assert np.array_equal(bits_of(y), bits_of(c["y"]))


def np_unpack(w_q, K, bits):
    """codes from the little-endian bitstream, by numpy's bit unpacking"""
    N = w_q.shape[0]
    bitsarr = np.unpackbits(np.ascontiguousarray(w_q).view(np.uint8).reshape(N, -1), axis=1, bitorder="little")
    bitsarr = bitsarr[:, :K * bits].reshape(N, K, bits).astype(np.uint32)
    return (bitsarr << np.arange(bits, dtype=np.uint32)).sum(axis=2)


def to_f64(a, dt):
    from oracle import oracle as O
    return (a if dt == F32 else O.to_f32(a, dt)).astype(np.float64)


@pytest.mark.parametrize("key", sorted(CASES))
def test_fixture_against_independent_restatement(oracle, key):
    c = CASES[key]
    M, K, N, bits, gs, xd, sbd = (int(v) for v in c["meta"])
    q = np_unpack(c["w_q"], K, bits).astype(np.float64)
    assert q.max() < 2 ** bits
    s = np.repeat(to_f64(c["s"], sbd), gs, axis=1)
    b = np.repeat(to_f64(c["b"], sbd), gs, axis=1)
    with np.errstate(invalid="ignore", over="ignore"):
        deq = (s * q + b).astype(np.float32)   # exact product and sum in float64, one rounding
    assert np.array_equal(np.isnan(deq), np.isnan(c["deq"]))
    fin = ~np.isnan(deq)
    assert np.array_equal(deq[fin].view(np.uint32), c["deq"][fin].view(np.uint32))
    rows = np.all(np.isfinite(c["deq"]), axis=1)
    exact = to_f64(c["x"], xd) @ c["deq"][rows].astype(np.float64).T
    got = c["y"][:, rows].astype(np.float64)
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()


def test_special_groups_follow_the_quantizer_rules(oracle):
    """the special case's groups: a constant group has scale 0 and codes 0;
    signed zeros quantize like zeros; a group holding inf or NaN has a
    non-finite scale or bias (its weights are not representable)"""
    c = CASES["b4_g32_special"]
    q = np_unpack(c["w_q"], 128, 4)
    assert c["s"][0, 0] == 0 and not q[0, :32].any()
    assert c["deq"][0, 0] == np.float32(0.375)
    assert np.all(c["deq"][0, 32:64] == 0)
    assert not np.isfinite(c["s"][3, 0]) or not np.isfinite(c["b"][3, 0])


def test_full_size_digests(oracle):
    import sys
    sys.path.insert(0, GOLD)
    from make_fixtures import DIGEST_CASES, digest_case
    with open(os.path.join(GOLD, "digests.json")) as f:
        want = json.load(f)
    for name, M, K, N, bits, gs, xd, sbd, outlier_frac in DIGEST_CASES:
        assert want[name]["outlier_frac"] == outlier_frac, name
        assert digest_case(M, K, N, bits, gs, xd, sbd, outlier_frac) == want[name]["sha256"], name
