"""Host runtime over the HIP plugin's C ABI: contexts, device buffers, and
the quantized ops, with numpy arrays on the host side.

This is plumbing for tests and the benchmark; the product is the plugin
library.  Every call goes through the vtable / quant-extension function
pointers the plugin exported, exactly as a C or Go embedder would call them,
and raises LuxError on a non-OK LuxBackendError.  There is no CPU fallback:
if the plugin or its GPU is missing, get_backend() raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import numpy as np

from . import abi
from .loader import LoadedBackend, PluginLoader

_ESZ = {abi.FLOAT32: 4, abi.FLOAT16: 2, abi.BFLOAT16: 2}
_NP = {abi.FLOAT32: np.float32, abi.FLOAT16: np.uint16, abi.BFLOAT16: np.uint16}


class LuxError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {abi.ERROR_NAMES.get(code, code)}")
        self.code = code


def _check(code: int, what: str) -> None:
    if code != abi.OK:
        raise LuxError(code, what)


_backend: Optional[LoadedBackend] = None


def get_backend(name: str = "hip") -> LoadedBackend:
    """Load the named plugin through the loader (LUX_GPU_BACKEND_PATH, then
    the default and in-tree plugin directories)."""
    global _backend
    if _backend is None:
        L = PluginLoader()
        if not L.load_backend(name):
            raise RuntimeError(
                f"backend '{name}' unavailable: libluxgpu_backend_{name}.so not found, "
                "or no gfx950 device (searched: " + ", ".join(L.search_paths) + ")")
        b = L.get_backend(name)
        if b.quant is None:
            raise RuntimeError(f"backend '{name}' has no quantized-matmul extension")
        _backend = b
    return _backend


class Buffer:
    def __init__(self, ctx: "Context", handle: int, nbytes: int):
        self.ctx, self.handle, self.nbytes = ctx, handle, nbytes

    def free(self) -> None:
        if self.handle:
            self.ctx.vt.buffer_free(self.ctx.handle, self.handle)
            self.handle = None

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(self.ctx.vt.buffer_copy_to_host(self.ctx.handle, self.handle,
                                               out.ctypes.data, out.nbytes), "buffer_copy_to_host")
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        _check(self.ctx.vt.buffer_copy_from_host(self.ctx.handle, self.handle,
                                                 a.ctypes.data, a.nbytes), "buffer_copy_from_host")


class Context:
    def __init__(self, device_index: int = 0, backend: Optional[LoadedBackend] = None):
        self.be = backend or get_backend()
        self.vt = self.be.vtbl
        self.q = self.be.quant
        self.handle = self.vt.create_context(device_index)
        if not self.handle:
            raise RuntimeError(f"create_context({device_index}) failed")

    def close(self) -> None:
        if self.handle:
            self.vt.destroy_context(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # --- buffers ---------------------------------------------------------
    def alloc(self, nbytes: int) -> Buffer:
        h = self.vt.buffer_alloc(self.handle, nbytes)
        if not h:
            raise LuxError(abi.ERR_OUT_OF_MEMORY, f"buffer_alloc({nbytes})")
        return Buffer(self, h, nbytes)

    def upload(self, a: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(a)
        h = self.vt.buffer_alloc_with_data(self.handle, a.ctypes.data, a.nbytes)
        if not h:
            raise LuxError(abi.ERR_OUT_OF_MEMORY, f"buffer_alloc_with_data({a.nbytes})")
        return Buffer(self, h, a.nbytes)

    def sync(self) -> None:
        _check(self.vt.sync(self.handle), "sync")

    def device_info(self) -> abi.DeviceInfo:
        info = abi.DeviceInfo()
        _check(self.vt.get_device_info(self.handle, ctypes.byref(info)), "get_device_info")
        return info

    @property
    def stream(self) -> int:
        return self.q.get_native_stream(self.handle)

    # --- quantized ops (asynchronous on the context stream) ---------------
    def quantized_matmul(self, x: Buffer, w_q: Buffer, scales: Buffer, biases: Buffer, out: Buffer,
                         M: int, K: int, N: int, group_size: int, bits: int, x_dtype: int,
                         sb_dtype: int, out_dtype: int, kernel: int = abi.KERNEL_AUTO) -> None:
        _check(self.q.op_quantized_matmul_ex(self.handle, x.handle, w_q.handle, scales.handle,
                                             biases.handle, out.handle, M, K, N, group_size, bits,
                                             x_dtype, sb_dtype, out_dtype, kernel),
               "op_quantized_matmul")

    def quantized_matmul_fused(self, x: Buffer, w_q: Buffer, scales: Buffer, biases: Buffer,
                               bias: Optional[Buffer], out: Buffer, M: int, K: int, N: int,
                               group_size: int, bits: int, x_dtype: int, sb_dtype: int,
                               bias_dtype: int, out_dtype: int, act: int = abi.ACT_NONE) -> None:
        """out = act(x . w_hat^T + bias), bias/act applied in fp32 in the kernel."""
        _check(self.q.op_quantized_matmul_fused(self.handle, x.handle, w_q.handle, scales.handle,
                                                biases.handle, bias.handle if bias else None,
                                                out.handle, M, K, N, group_size, bits, x_dtype,
                                                sb_dtype, bias_dtype, out_dtype, act),
               "op_quantized_matmul_fused")

    def load_linear(self, path: str, prefix: str, group_size: int = 0, bits: int = 0) -> "LinearLayer":
        """A quantized linear layer from a safetensors file, on this context's
        device (group_size / bits 0: from the file's metadata)."""
        lin = abi.Linear()
        _check(self.q.linear_load(self.handle, path.encode(), prefix.encode(), group_size, bits,
                                  ctypes.byref(lin)), "linear_load")
        return LinearLayer(self, lin)

    def dequantize(self, w_q: Buffer, scales: Buffer, biases: Buffer, out: Buffer, N: int, K: int,
                   group_size: int, bits: int, sb_dtype: int, out_dtype: int) -> None:
        _check(self.q.op_dequantize(self.handle, w_q.handle, scales.handle, biases.handle,
                                    out.handle, N, K, group_size, bits, sb_dtype, out_dtype),
               "op_dequantize")

    def quantize(self, w: Buffer, w_q: Buffer, scales: Buffer, biases: Buffer, N: int, K: int,
                 group_size: int, bits: int, w_dtype: int, sb_dtype: int) -> None:
        _check(self.q.op_quantize(self.handle, w.handle, w_q.handle, scales.handle, biases.handle,
                                  N, K, group_size, bits, w_dtype, sb_dtype), "op_quantize")

    def select_kernel(self, M, K, N, group_size, bits, x_dtype, sb_dtype=None) -> int:
        """The kernel AUTO runs for this shape; sb_dtype defaults to x_dtype."""
        return self.q.select_kernel(M, K, N, group_size, bits, x_dtype,
                                    x_dtype if sb_dtype is None else sb_dtype)

    def kernel_name(self, M, K, N, group_size, bits, x_dtype, sb_dtype=None, out_dtype=None,
                    kernel: int = abi.KERNEL_AUTO) -> Optional[str]:
        """The gfx950 kernel op_quantized_matmul_ex launches for this shape
        (lux_gpu_quantized_matmul_kernel_name: a dry run of the dispatch);
        None where the op would fail.  sb/out dtypes default to x_dtype."""
        f = getattr(self.be.handle, "lux_gpu_quantized_matmul_kernel_name", None)
        if f is None:
            return None
        f.restype = ctypes.c_char_p
        f.argtypes = [ctypes.c_int] * 9
        sb = x_dtype if sb_dtype is None else sb_dtype
        r = f(M, K, N, group_size, bits, x_dtype, sb, sb if out_dtype is None else out_dtype, kernel)
        return None if r is None else r.decode()

    # base f32 tensor ops (vtable slots, as the reference core calls them)
    def binary_f32(self, op: str, a: Buffer, b: Buffer, out: Buffer, n: int) -> None:
        fn = getattr(self.vt, f"op_{op}_f32")
        if not fn:
            raise LuxError(abi.ERR_NOT_SUPPORTED, f"op_{op}_f32")
        _check(fn(self.handle, a.handle, b.handle, out.handle, n), f"op_{op}_f32")

    def matmul_f32(self, a: Buffer, b: Buffer, out: Buffer, M: int, K: int, N: int) -> None:
        _check(self.vt.op_matmul_f32(self.handle, a.handle, b.handle, out.handle, M, K, N), "op_matmul_f32")

    def transpose_f32(self, a: Buffer, out: Buffer, rows: int, cols: int) -> None:
        _check(self.vt.op_transpose_f32(self.handle, a.handle, out.handle, rows, cols), "op_transpose_f32")


class LinearLayer:
    """Device buffers of one quantized linear layer (lux_quant_linear)."""

    def __init__(self, ctx: Context, lin: "abi.Linear"):
        self.ctx, self.lin = ctx, lin
        i = lin.info
        self.N, self.K, self.group_size, self.bits = i.N, i.K, i.group_size, i.bits
        self.sb_dtype, self.bias_dtype, self.has_bias = i.sb_dtype, i.bias_dtype, bool(i.has_bias)
        self.w_q = Buffer(ctx, lin.w_q, i.weight_bytes)
        self.scales = Buffer(ctx, lin.scales, i.scales_bytes)
        self.biases = Buffer(ctx, lin.biases, i.biases_bytes)
        self.bias = Buffer(ctx, lin.bias, i.bias_bytes) if lin.bias else None

    def __call__(self, x: Buffer, out: Buffer, M: int, x_dtype: int, out_dtype: int,
                 act: int = abi.ACT_NONE, use_bias: bool = True) -> None:
        """out[M, N] = act(x . W^T + bias): the fused op, with the file's bias if it has one."""
        bias = self.bias if (use_bias and self.has_bias) else None
        self.ctx.quantized_matmul_fused(x, self.w_q, self.scales, self.biases, bias, out, M, self.K,
                                        self.N, self.group_size, self.bits, x_dtype, self.sb_dtype,
                                        self.bias_dtype, out_dtype, act)

    def free(self) -> None:
        if self.lin is not None:
            self.ctx.q.linear_free(self.ctx.handle, ctypes.byref(self.lin))
            self.lin = None
            for b in (self.w_q, self.scales, self.biases, self.bias):
                if b:
                    b.handle = None


def describe_linear(quant: "abi.QuantVtbl", path: str, prefix: str, group_size: int = 0,
                    bits: int = 0) -> "abi.LinearInfo":
    """Host-only header parse (no device needed): the layer's shapes and offsets."""
    info = abi.LinearInfo()
    _check(quant.linear_describe(path.encode(), prefix.encode(), group_size, bits, ctypes.byref(info)),
           "linear_describe")
    return info


def esize(dtype: int) -> int:
    return _ESZ[dtype]


def np_dtype(dtype: int):
    return _NP[dtype]


def run_quantized_matmul(ctx: Context, x: np.ndarray, w_q: np.ndarray, scales: np.ndarray,
                         biases: np.ndarray, M: int, K: int, N: int, group_size: int, bits: int,
                         x_dtype: int, sb_dtype: int, out_dtype: int,
                         kernel: int = abi.KERNEL_AUTO) -> np.ndarray:
    """Upload, run one quantized matmul, download.  Host arrays in, host array out."""
    bufs = [ctx.upload(a) for a in (x, w_q, scales, biases)]
    out = ctx.alloc(max(1, M * N * esize(out_dtype)))
    try:
        ctx.quantized_matmul(*bufs, out, M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype,
                             kernel)
        return out.download(np_dtype(out_dtype), (M, N))
    finally:
        for b in bufs + [out]:
            b.free()


def run_dequantize(ctx: Context, w_q, scales, biases, K: int, group_size: int, bits: int,
                   sb_dtype: int, out_dtype: int) -> np.ndarray:
    N = w_q.shape[0]
    bufs = [ctx.upload(a) for a in (w_q, scales, biases)]
    out = ctx.alloc(max(1, N * K * esize(out_dtype)))
    try:
        ctx.dequantize(*bufs, out, N, K, group_size, bits, sb_dtype, out_dtype)
        return out.download(np_dtype(out_dtype), (N, K))
    finally:
        for b in bufs + [out]:
            b.free()


def run_quantize(ctx: Context, w: np.ndarray, group_size: int, bits: int, w_dtype: int,
                 sb_dtype: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    N, K = w.shape
    G = K // group_size
    wb = ctx.upload(w)
    wq = ctx.alloc(N * K * bits // 8)
    s = ctx.alloc(N * G * esize(sb_dtype))
    b = ctx.alloc(N * G * esize(sb_dtype))
    try:
        ctx.quantize(wb, wq, s, b, N, K, group_size, bits, w_dtype, sb_dtype)
        return (wq.download(np.uint32, (N, K * bits // 32)),
                s.download(np_dtype(sb_dtype), (N, G)), b.download(np_dtype(sb_dtype), (N, G)))
    finally:
        for x in (wb, wq, s, b):
            x.free()
