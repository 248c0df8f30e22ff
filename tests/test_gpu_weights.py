"""Quantized linear layers from safetensors files on the GPU: linear_load
puts the file's tensors on the device unchanged (bit-exact dequantization
against the oracle), and the loaded layer runs the fused op with the file's
output bias.  The round trip starts from the GPU quantizer, so a layer
quantized on the device, saved and loaded again computes the same output.
"""
import numpy as np
import pytest

from qmm_util import BF16, F16, F32, check_output

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,bits,gs,sbd,xd", [
    (14336, 4096, 4, 64, F16, F16),   # configs[1] layer
    (300, 768, 3, 128, BF16, BF16),
    (96, 512, 6, 32, F32, F16),
])
def test_quantize_save_load_run(ctx, oracle, tmp_path, N, K, bits, gs, sbd, xd):
    from safetensors.numpy import save_file
    from mlx_amd import abi, runtime
    O = oracle
    w = O.rng_normal(N * K, 7000 + bits, 0.0, 0.02).reshape(N, K)
    print(f"[case] weights N={N} K={K} b={bits} g={gs} sb={sbd}", flush=True)
    w_q, s, b = runtime.run_quantize(ctx, w, gs, bits, F32, sbd)
    bias = O.rng_normal(N, 7100 + N, 0.0, 0.5).astype(np.float32)
    # 16-bit scales travel as uint16 bit patterns; the file names their dtype
    path = str(tmp_path / "layer.safetensors")
    sb_np = {F32: s, F16: s.view(np.float16), BF16: s}
    bi_np = {F32: b, F16: b.view(np.float16), BF16: b}
    tensors = {"blk.0.mlp.weight": w_q, "blk.0.mlp.scales": sb_np[sbd], "blk.0.mlp.biases": bi_np[sbd],
               "blk.0.mlp.bias": bias}
    if sbd == BF16:
        _save_with_bf16(path, tensors, ["blk.0.mlp.scales", "blk.0.mlp.biases"], {"bits": str(bits)})
        gs_arg = gs
    else:
        save_file(tensors, path, metadata={"bits": str(bits), "group_size": str(gs)})
        gs_arg = 0
    lin = ctx.load_linear(path, "blk.0.mlp", gs_arg, 0)
    try:
        assert (lin.N, lin.K, lin.bits, lin.group_size, lin.sb_dtype, lin.has_bias) == (N, K, bits, gs, sbd, True)
        # the device copy is the file: dequantization bit-equal to the oracle's
        rows = min(N, 512)
        out = ctx.alloc(N * K * 4)
        ctx.dequantize(lin.w_q, lin.scales, lin.biases, out, N, K, gs, bits, sbd, F32)
        got = out.download(np.float32, (N, K))[:rows]
        out.free()
        assert np.array_equal(got.view(np.uint32),
                              O.dequantize(w_q[:rows], s[:rows], b[:rows], K, gs, bits, sbd, F32).view(np.uint32))
        # fused op with the file's bias, against the oracle on the host arrays
        M = 1 if N > 4096 else 3
        x = O.from_f32(O.rng_normal(M * K, 7200, 0.0, 1.0).reshape(M, K), xd)
        X = ctx.upload(x)
        Y = ctx.alloc(M * N * 4)
        lin(X, Y, M, xd, F32, act=abi.ACT_SILU)
        y = Y.download(np.float32, (M, N))
        X.free()
        Y.free()
        gemm = ctx.select_kernel(M, K, N, gs, bits, xd, sbd) == abi.KERNEL_GEMM
        acc = O.quantized_matmul(x, w_q, s, b, M, K, N, gs, bits, xd, sbd, F32, variant="omp",
                                 w_round=xd if gemm else F32)
        check_output(O, y, O.fused_epilogue(acc, bias, F32, abi.ACT_SILU, F32), F32, "loaded layer")
    finally:
        lin.free()


def _save_with_bf16(path, tensors, bf16_names, metadata):
    """safetensors.numpy has no bfloat16: write the file directly."""
    import json
    import struct
    dt = {np.dtype(np.uint32): "U32", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}
    header, off, blobs = {}, 0, []
    for k, a in tensors.items():
        a = np.ascontiguousarray(a)
        header[k] = {"dtype": "BF16" if k in bf16_names else dt[a.dtype], "shape": list(a.shape),
                     "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
        blobs.append(a.tobytes())
    header["__metadata__"] = metadata
    js = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)) + js + b"".join(blobs))


def test_load_errors_leave_nothing_allocated(ctx, tmp_path):
    from mlx_amd import abi, runtime
    p = str(tmp_path / "none.safetensors")
    with pytest.raises(runtime.LuxError) as e:
        ctx.load_linear(p, "w", 64, 4)
    assert e.value.code == abi.ERR_INVALID_ARGUMENT
    # a layer whose parameters disagree with the weight: rejected before any allocation
    from safetensors.numpy import save_file
    save_file({"w.weight": np.zeros((8, 32), np.uint32), "w.scales": np.ones((8, 4), np.float16),
               "w.biases": np.zeros((8, 4), np.float16)}, p)
    with pytest.raises(runtime.LuxError) as e:
        ctx.load_linear(p, "w", 64, 8)
    assert e.value.code == abi.ERR_INVALID_ARGUMENT
    lin = ctx.load_linear(p, "w", 64, 4)
    assert (lin.N, lin.K, lin.has_bias, lin.bias) == (8, 256, False, None)
    lin.free()
    lin.free()  # a second free is a no-op
