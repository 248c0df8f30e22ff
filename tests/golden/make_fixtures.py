"""Writes the golden fixtures of the quantized-matmul path (test data only).

    python tests/golden/make_fixtures.py          # rewrite golden.npz + digests.json

golden.npz -- small cases computed by the CPU oracle (oracle/lux_cpu_quant.c):
  for each case key k:
    k/w      fp32 weights [N, K] (including special values where named)
    k/w_q    packed codes uint32 [N, K*bits/32]     (quantize)
    k/s, k/b scales, biases [N, K/g] (sb dtype; 16-bit types as uint16 bits)
    k/deq    dequantized weights, fp32 [N, K]        (dequantize, fmaf form)
    k/x      activations [M, K] (x dtype; 16-bit as uint16 bits)
    k/y      x . deq^T, fp32 [M, N] (the oracle's ascending-k fp32 sums)
    k/meta   int32 [M, K, N, bits, group, x_dtype, sb_dtype]
digests.json -- SHA-256 of the full-size synthetic tensors each BASELINE
config uses (oracle make_problem, seed 1): pins the generator and the
quantizer at full size without committing hundreds of megabytes.
The fixtures are data: they hold no code of the reference.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

F32, F16, BF16 = 0, 1, 2

# (key, M, K, N, bits, group, x dtype, sb dtype, special)
CASES = [
    ("b2_g32_f16", 3, 128, 5, 2, 32, F16, F16, None),
    ("b3_g64_bf16", 2, 192, 6, 3, 64, BF16, BF16, None),
    ("b4_g64_f32", 1, 256, 7, 4, 64, F32, F32, None),
    ("b4_g32_f16", 4, 128, 9, 4, 32, F16, F32, None),
    ("b4_g128_bf16", 2, 256, 4, 4, 128, BF16, BF16, None),
    ("b5_g32_f32", 2, 160, 3, 5, 32, F32, F16, None),
    ("b6_g64_f16", 3, 128, 5, 6, 64, F16, F16, None),
    ("b8_g128_bf16", 2, 256, 3, 8, 128, BF16, BF16, None),
    # special groups: constant (scale 0), +-0, a huge outlier, +-inf and NaN
    ("b4_g32_special", 2, 128, 4, 4, 32, F32, F32, "special"),
]

# full-size synthetic inputs of the configs, seed 1
# (name, M, K, N, bits, group, x dtype, scale dtype, fraction of W entries
# scaled x20: configs[4]'s outliers)
DIGEST_CASES = [
    ("c0", 1, 4096, 4096, 4, 64, F32, F32, 0.0),
    ("c1", 8, 4096, 14336, 4, 64, F16, F16, 0.0),
    ("c2", 32, 8192, 8192, 8, 128, BF16, BF16, 0.0),
    ("c3_n4096", 2048, 4096, 4096, 4, 64, BF16, BF16, 0.0),
    ("c4_b3", 64, 4096, 11008, 3, 64, F16, F16, 0.01),
    ("c4_b6", 64, 4096, 11008, 6, 64, F16, F16, 0.01),
]


def special_weights(N, K):
    from oracle import oracle as O
    w = O.rng_normal(N * K, 77, 0.0, 0.02).reshape(N, K)
    w[0, 0:32] = 0.375             # constant group: scale 0, every code 0
    w[0, 32:48] = -0.0             # signed zeros in a group
    w[0, 48:64] = 0.0
    w[1, 64] = 20.0                # outlier stretches its group's scale
    w[2, 96:128] = -1.5e-6         # tiny constant group
    w[3, 0] = np.inf               # non-finite values: the group's scale and
    w[3, 40] = -np.inf             # bias follow the quantizer's rules
    w[3, 70] = np.nan
    return w


def build_case(key, M, K, N, bits, gs, xd, sbd, special):
    from oracle import oracle as O
    if special == "special":
        w = special_weights(N, K)
        x = O.from_f32(O.rng_normal(M * K, 78).reshape(M, K), xd)
        w_q, s, b = O.quantize(w, gs, bits, sbd)
    else:
        x, w_q, s, b, w = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=500 + len(key))
    deq = O.dequantize(w_q, s, b, K, gs, bits, sbd)
    y = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32)
    return {"w": w.astype(np.float32), "w_q": w_q, "s": s, "b": b, "deq": deq, "x": x, "y": y,
            "meta": np.array([M, K, N, bits, gs, xd, sbd], np.int32)}


def digest_case(M, K, N, bits, gs, xd, sbd, outlier_frac=0.0):
    from oracle import oracle as O
    x, w_q, s, b, _ = O.make_problem(M, K, N, bits, gs, xd, sbd, seed=1, outlier_frac=outlier_frac)
    return {name: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
            for name, a in (("x", x), ("w_q", w_q), ("scales", s), ("biases", b))}


def main(digests_only=False):
    from oracle import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    if not digests_only:
        arrays = {}
        for key, *c in CASES:
            for name, a in build_case(key, *c).items():
                arrays[f"{key}/{name}"] = a
        np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    digests = {name: {"shape": [M, K, N], "bits": bits, "group_size": gs, "x_dtype": xd, "sb_dtype": sbd,
                      "seed": 1, "outlier_frac": of, "sha256": digest_case(M, K, N, bits, gs, xd, sbd, of)}
               for name, M, K, N, bits, gs, xd, sbd, of in DIGEST_CASES}
    with open(os.path.join(HERE, "digests.json"), "w") as f:
        json.dump(digests, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {len(CASES)} cases and {len(digests)} digests")


if __name__ == "__main__":
    main(digests_only="--digests-only" in sys.argv)
