"""Quantized linear layers in safetensors files, on the CPU: the plugin's
header parser (quant table slot linear_describe, host code, no device)
against files written here.

The writer below is checked against the safetensors library itself (its
files load there with the same arrays, and the library's files parse
here), so the layout tests do not rest on a writer of our own alone.
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

F32, F16, BF16 = 0, 1, 2
INVALID, NOT_SUPPORTED = 1, 3
_NP_DT = {np.dtype(np.uint32): "U32", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}


def write_st(path, tensors, metadata=None, dtypes=None, pad=0):
    """A safetensors file: {name: ndarray}; dtypes overrides the dtype string
    (e.g. "BF16" for uint16 bit patterns)."""
    dtypes = dtypes or {}
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        dt = dtypes.get(name, _NP_DT.get(a.dtype))
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    if metadata is not None:
        header["__metadata__"] = metadata
    js = json.dumps(header).encode() + b" " * pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        for b in blobs:
            f.write(b)


@pytest.fixture(scope="module")
def quant():
    import mlx_amd
    from mlx_amd import abi
    assert mlx_amd.plugin_built(), "plugin not built: run __graft_entry__.build()"
    lib = ctypes.CDLL(mlx_amd.PLUGIN_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    qinit = abi.QUANT_INIT_FN(("lux_gpu_backend_quant_init", lib))
    p = ctypes.POINTER(abi.QuantVtbl)()
    assert qinit(ctypes.byref(p))
    return p.contents


def describe(quant, path, prefix, gs=0, bits=0):
    from mlx_amd import abi
    info = abi.LinearInfo()
    rc = quant.linear_describe(str(path).encode(), prefix.encode(), gs, bits, ctypes.byref(info))
    return rc, info


def layer(N=24, K=256, bits=4, gs=64, sb=np.float16, bias=True, seed=0):
    rng = np.random.default_rng(seed)
    t = {"w.weight": rng.integers(0, 2**32, (N, K * bits // 32), dtype=np.uint32),
         "w.scales": rng.standard_normal((N, K // gs)).astype(sb),
         "w.biases": rng.standard_normal((N, K // gs)).astype(sb)}
    if bias:
        t["w.bias"] = rng.standard_normal(N).astype(np.float32)
    return t


def test_writer_matches_safetensors_library(tmp_path):
    from safetensors.numpy import load_file, save_file
    t = layer()
    write_st(tmp_path / "a.safetensors", t)
    back = load_file(str(tmp_path / "a.safetensors"))
    assert set(back) == set(t) and all(np.array_equal(back[k], t[k]) for k in t)
    save_file(t, str(tmp_path / "b.safetensors"), metadata={"bits": "4", "group_size": "64"})
    back = load_file(str(tmp_path / "b.safetensors"))
    assert all(np.array_equal(back[k], t[k]) for k in t)


@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 64), (4, 64), (5, 128), (6, 32), (8, 128)])
def test_describe_offsets_and_shapes(quant, tmp_path, bits, gs):
    N, K = 24, 768 if bits in (3, 5, 6) else 512
    t = layer(N, K, bits, gs, seed=bits)
    p = tmp_path / "m.safetensors"
    write_st(p, t, pad=5)
    rc, i = describe(quant, p, "w", gs, bits)
    assert rc == 0
    assert (i.N, i.K, i.group_size, i.bits, i.sb_dtype, i.has_bias, i.bias_dtype) == (N, K, gs, bits, F16, 1, F32)
    raw = open(p, "rb").read()
    for name, off, nb in [("w.weight", i.weight_offset, i.weight_bytes), ("w.scales", i.scales_offset, i.scales_bytes),
                          ("w.biases", i.biases_offset, i.biases_bytes), ("w.bias", i.bias_offset, i.bias_bytes)]:
        assert raw[off:off + nb] == t[name].tobytes(), name


def test_library_written_file_and_metadata(quant, tmp_path):
    """A file from safetensors.numpy.save_file (its own header order and
    padding); bits / group size from __metadata__, per-layer entries first."""
    from safetensors.numpy import save_file
    t = layer(N=40, K=384, bits=3, gs=128, sb=np.float32, bias=False)
    p = tmp_path / "lib.safetensors"
    save_file(t, str(p), metadata={"bits": "8", "group_size": "32", "w.bits": "3", "w.group_size": "128"})
    rc, i = describe(quant, p, "w")
    assert rc == 0 and (i.N, i.K, i.bits, i.group_size, i.sb_dtype, i.has_bias) == (40, 384, 3, 128, F32, 0)
    raw = open(p, "rb").read()
    assert raw[i.weight_offset:i.weight_offset + i.weight_bytes] == t["w.weight"].tobytes()
    # global entries when there is no per-layer one
    save_file(t, str(p), metadata={"bits": "3", "group_size": "128"})
    assert describe(quant, p, "w")[0] == 0
    # arguments win over the file
    rc, i = describe(quant, p, "w", 64, 0)
    assert rc == INVALID  # K = 3 * 64 = 192: the weight's 36 words per row do not match


def test_bf16_scales_and_bias(quant, tmp_path):
    t = layer(sb=np.float16)
    t["w.scales"] = t["w.scales"].view(np.uint16)
    t["w.biases"] = t["w.biases"].view(np.uint16)
    t["w.bias"] = np.zeros(24, np.uint16)
    p = tmp_path / "bf.safetensors"
    write_st(p, t, dtypes={"w.scales": "BF16", "w.biases": "BF16", "w.bias": "BF16"})
    rc, i = describe(quant, p, "w", 64, 4)
    assert rc == 0 and i.sb_dtype == BF16 and i.bias_dtype == BF16


def test_describe_errors(quant, tmp_path):
    p = tmp_path / "e.safetensors"
    good = layer()

    def rc_of(tensors, gs=64, bits=4, prefix="w", **kw):
        write_st(p, tensors, **kw)
        return describe(quant, p, prefix, gs, bits)[0]

    assert rc_of(good) == 0
    assert rc_of(good, prefix="v") == INVALID                       # no such layer
    assert rc_of({k: v for k, v in good.items() if k != "w.biases"}) == INVALID
    assert rc_of(good, gs=0, bits=0) == INVALID                     # no parameters anywhere
    assert rc_of(good, bits=7) == NOT_SUPPORTED
    assert rc_of(good, gs=48) == NOT_SUPPORTED
    assert rc_of(good, bits=8) == INVALID                           # weight words disagree with K
    bad = dict(good, **{"w.biases": good["w.biases"].astype(np.float32)})
    assert rc_of(bad) == INVALID                                    # scales / biases dtypes differ
    bad = dict(good, **{"w.scales": good["w.scales"][:-1], "w.biases": good["w.biases"][:-1]})
    assert rc_of(bad) == INVALID                                    # N disagrees
    bad = dict(good, **{"w.bias": np.zeros(23, np.float32)})
    assert rc_of(bad) == INVALID                                    # bias length
    bad = dict(good, **{"w.weight": good["w.weight"].view(np.float32)})
    assert rc_of(bad) == NOT_SUPPORTED                              # weight not U32
    assert rc_of(good, dtypes={"w.bias": "F64"}) == NOT_SUPPORTED
    # malformed files
    write_st(p, good)
    raw = bytearray(open(p, "rb").read())
    for mutate in (lambda r: r[:7],                                  # shorter than the length field
                   lambda r: r[:len(r) - 1],                         # data cut short
                   lambda r: struct.pack("<Q", 2**40) + r[8:],       # header length past the end
                   lambda r: r[:8] + b"[" + r[9:],                   # header not an object
                   lambda r: r[:8] + r[8:].replace(b'"data_offsets"', b'"data_offsetz"', 1)):
        open(p, "wb").write(bytes(mutate(raw)))
        assert describe(quant, p, "w", 64, 4)[0] == INVALID
    # offsets out of range / overlapping a shape of another size
    h = json.loads(bytes(raw[8:8 + struct.unpack("<Q", raw[:8])[0]]))
    h["w.bias"]["data_offsets"][1] += 4
    js = json.dumps(h).encode()
    open(p, "wb").write(struct.pack("<Q", len(js)) + js + bytes(raw[8 + struct.unpack("<Q", raw[:8])[0]:]))
    assert describe(quant, p, "w", 64, 4)[0] == INVALID
    assert describe(quant, tmp_path / "missing.safetensors", "w", 64, 4)[0] == INVALID


def test_json_escapes_in_names(quant, tmp_path):
    """Tensor names with escapes (\\u, surrogate pairs, quotes) parse to the
    same UTF-8 names the prefix is matched against."""
    pre = 'layers.0/é\U0001F600"q"'
    t = {pre + ".weight": np.zeros((4, 32), np.uint32), pre + ".scales": np.ones((4, 4), np.float16),
         pre + ".biases": np.zeros((4, 4), np.float16)}
    p = tmp_path / "u.safetensors"
    header, off, blobs = {}, 0, []
    for k, a in t.items():
        header[k] = {"dtype": _NP_DT[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
        blobs.append(a.tobytes())
    js = json.dumps(header, ensure_ascii=True).encode()   # \\uXXXX escapes, surrogate pair for the emoji
    assert b"\\ud83d\\ude00" in js
    open(p, "wb").write(struct.pack("<Q", len(js)) + js + b"".join(blobs))
    from mlx_amd import abi
    info = abi.LinearInfo()
    rc = quant.linear_describe(str(p).encode(), pre.encode("utf-8"), 64, 4, ctypes.byref(info))
    assert rc == 0 and (info.N, info.K) == (4, 256)
