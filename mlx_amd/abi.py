"""ctypes mirror of the Lux GPU backend plugin ABI v2 and the quant extension.

Layout follows include/lux_gpu_backend_abi.h (itself layout-identical to the
reference include/lux/gpu/backend_plugin.h:82-394): a 64-slot function table
(512 bytes on LP64), a 40-byte descriptor and a 48-byte device-info struct.
Only the slots the HIP plugin fills get precise prototypes; the rest are
opaque pointers so that the struct size and offsets stay exact.
"""
from __future__ import annotations

import ctypes as C

ABI_VERSION = 2                      # backend_plugin.h:24
INIT_SYMBOL = b"lux_gpu_backend_init"  # backend_plugin.h:426
QUANT_INIT_SYMBOL = b"lux_gpu_backend_quant_init"
QUANT_EXT_VERSION = 1

# LuxBackendDtype (backend_plugin.h:38-47)
FLOAT32, FLOAT16, BFLOAT16, INT32, INT64, UINT32, UINT64, BOOL = range(8)

# LuxBackendError (backend_plugin.h:49-56)
OK, ERR_INVALID_ARGUMENT, ERR_OUT_OF_MEMORY, ERR_NOT_SUPPORTED, ERR_DEVICE_LOST, ERR_INTERNAL = range(6)
ERROR_NAMES = {
    OK: "OK",
    ERR_INVALID_ARGUMENT: "INVALID_ARGUMENT",
    ERR_OUT_OF_MEMORY: "OUT_OF_MEMORY",
    ERR_NOT_SUPPORTED: "NOT_SUPPORTED",
    ERR_DEVICE_LOST: "DEVICE_LOST",
    ERR_INTERNAL: "INTERNAL",
}

# LuxQuantKernel
KERNEL_AUTO, KERNEL_GEMV, KERNEL_GEMM = 0, 1, 2

# capability bits (backend_plugin.h:397-415)
CAP_TENSOR_OPS = 1 << 0
CAP_MATMUL = 1 << 1
CAP_UNIFIED_MEMORY = 1 << 5

Ctx = C.c_void_p
Buf = C.c_void_p
Err = C.c_int


class DeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("vendor", C.c_char_p),
        ("memory_total", C.c_uint64),
        ("memory_available", C.c_uint64),
        ("compute_units", C.c_int),
        ("max_workgroup_size", C.c_int),
        ("is_discrete", C.c_bool),
        ("is_unified_memory", C.c_bool),
    ]


CREATE_CONTEXT = C.CFUNCTYPE(Ctx, C.c_int)
DESTROY_CONTEXT = C.CFUNCTYPE(None, Ctx)
GET_DEVICE_COUNT = C.CFUNCTYPE(Err, C.POINTER(C.c_int))
GET_DEVICE_INFO = C.CFUNCTYPE(Err, Ctx, C.POINTER(DeviceInfo))
SYNC = C.CFUNCTYPE(Err, Ctx)
BUFFER_ALLOC = C.CFUNCTYPE(Buf, Ctx, C.c_size_t)
BUFFER_ALLOC_WITH_DATA = C.CFUNCTYPE(Buf, Ctx, C.c_void_p, C.c_size_t)
BUFFER_FREE = C.CFUNCTYPE(None, Ctx, Buf)
BUFFER_COPY_TO_HOST = C.CFUNCTYPE(Err, Ctx, Buf, C.c_void_p, C.c_size_t)
BUFFER_COPY_FROM_HOST = C.CFUNCTYPE(Err, Ctx, Buf, C.c_void_p, C.c_size_t)
BUFFER_GET_HOST_PTR = C.CFUNCTYPE(C.c_void_p, Ctx, Buf)
OP_MATMUL_F32 = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, C.c_int, C.c_int, C.c_int)
OP_BINARY_F32 = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, C.c_size_t)
OP_TRANSPOSE_F32 = C.CFUNCTYPE(Err, Ctx, Buf, Buf, C.c_int, C.c_int)

# slot index -> (name, prototype or None).  Slot order is the ABI
# (backend_plugin.h:82-380; probed offsets in SURVEY Appendix A).
_SLOT_NAMES = [
    "create_context", "destroy_context", "get_device_count", "get_device_info", "sync",
    "buffer_alloc", "buffer_alloc_with_data", "buffer_free", "buffer_copy_to_host",
    "buffer_copy_from_host", "buffer_get_host_ptr", "kernel_load", "kernel_load_binary",
    "kernel_destroy", "kernel_dispatch", "op_add_f32", "op_sub_f32", "op_mul_f32", "op_div_f32",
    "op_matmul_f32", "op_transpose_f32", "op_reduce_sum_f32", "op_reduce_max_f32",
    "op_reduce_min_f32", "op_reduce_mean_f32", "op_reduce_sum_axis_f32", "op_reduce_max_axis_f32",
    "op_softmax_f32", "op_log_softmax_f32", "op_exp_f32", "op_log_f32", "op_sqrt_f32",
    "op_neg_f32", "op_abs_f32", "op_tanh_f32", "op_sigmoid_f32", "op_relu_f32", "op_gelu_f32",
    "op_copy_f32", "op_layer_norm_f32", "op_rms_norm_f32", "op_ntt_forward", "op_ntt_inverse",
    "op_msm", "op_poly_mul", "op_tfhe_bootstrap", "op_tfhe_keyswitch", "op_blind_rotate",
    "op_sample_extract", "op_sample_ntt", "op_poseidon2_hash", "op_blake3_hash",
    "op_bls12_381_add", "op_bls12_381_mul", "op_bls12_381_pairing", "op_bn254_add",
    "op_bn254_mul", "op_kzg_commit", "op_kzg_open", "op_kzg_verify",
]
assert len(_SLOT_NAMES) == 60

_PROTOS = {
    "create_context": CREATE_CONTEXT,
    "destroy_context": DESTROY_CONTEXT,
    "get_device_count": GET_DEVICE_COUNT,
    "get_device_info": GET_DEVICE_INFO,
    "sync": SYNC,
    "buffer_alloc": BUFFER_ALLOC,
    "buffer_alloc_with_data": BUFFER_ALLOC_WITH_DATA,
    "buffer_free": BUFFER_FREE,
    "buffer_copy_to_host": BUFFER_COPY_TO_HOST,
    "buffer_copy_from_host": BUFFER_COPY_FROM_HOST,
    "buffer_get_host_ptr": BUFFER_GET_HOST_PTR,
    "op_matmul_f32": OP_MATMUL_F32,
    "op_add_f32": OP_BINARY_F32,
    "op_sub_f32": OP_BINARY_F32,
    "op_mul_f32": OP_BINARY_F32,
    "op_div_f32": OP_BINARY_F32,
    "op_transpose_f32": OP_TRANSPOSE_F32,
}


class BackendVtbl(C.Structure):
    _fields_ = [(n, _PROTOS.get(n, C.c_void_p)) for n in _SLOT_NAMES] + [("_reserved", C.c_void_p * 4)]


class BackendDesc(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("backend_name", C.c_char_p),
        ("backend_version", C.c_char_p),
        ("capabilities", C.c_uint32),
        ("vtbl", C.POINTER(BackendVtbl)),
    ]


INIT_FN = C.CFUNCTYPE(C.c_bool, C.POINTER(BackendDesc))

_I = C.c_int
OP_QMM = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, Buf, Buf, _I, _I, _I, _I, _I, _I, _I, _I)
OP_QMM_EX = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, Buf, Buf, _I, _I, _I, _I, _I, _I, _I, _I, _I)
OP_DEQUANT = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, Buf, _I, _I, _I, _I, _I, _I)
OP_QUANT = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, Buf, _I, _I, _I, _I, _I, _I)
GET_NATIVE_STREAM = C.CFUNCTYPE(C.c_void_p, Ctx)
SELECT_KERNEL = C.CFUNCTYPE(_I, _I, _I, _I, _I, _I, _I, _I)
# ctx, x, w_q, scales, biases, bias, out, M, K, N, group_size, bits, x_dt, sb_dt, bias_dt, out_dt, act
OP_QMM_FUSED = C.CFUNCTYPE(Err, Ctx, Buf, Buf, Buf, Buf, Buf, Buf, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I)
ACT_NONE, ACT_RELU, ACT_SILU, ACT_GELU = 0, 1, 2, 3


class LinearInfo(C.Structure):
    """lux_quant_linear_info: a quantized linear layer in a safetensors file."""
    _fields_ = [("N", C.c_int32), ("K", C.c_int32), ("group_size", C.c_int32), ("bits", C.c_int32),
                ("sb_dtype", C.c_int), ("bias_dtype", C.c_int), ("has_bias", C.c_int32), ("_pad", C.c_int32),
                ("weight_offset", C.c_uint64), ("weight_bytes", C.c_uint64),
                ("scales_offset", C.c_uint64), ("scales_bytes", C.c_uint64),
                ("biases_offset", C.c_uint64), ("biases_bytes", C.c_uint64),
                ("bias_offset", C.c_uint64), ("bias_bytes", C.c_uint64)]


class Linear(C.Structure):
    """lux_quant_linear: the layer's device buffers after linear_load."""
    _fields_ = [("info", LinearInfo), ("w_q", Buf), ("scales", Buf), ("biases", Buf), ("bias", Buf)]


LINEAR_DESCRIBE = C.CFUNCTYPE(Err, C.c_char_p, C.c_char_p, _I, _I, C.POINTER(LinearInfo))
LINEAR_LOAD = C.CFUNCTYPE(Err, Ctx, C.c_char_p, C.c_char_p, _I, _I, C.POINTER(Linear))
LINEAR_FREE = C.CFUNCTYPE(None, Ctx, C.POINTER(Linear))


class QuantVtbl(C.Structure):
    _fields_ = [
        ("ext_version", C.c_uint32),
        ("struct_size", C.c_uint32),
        ("op_quantized_matmul", OP_QMM),
        ("op_dequantize", OP_DEQUANT),
        ("op_quantize", OP_QUANT),
        ("op_quantized_matmul_ex", OP_QMM_EX),
        ("get_native_stream", GET_NATIVE_STREAM),
        ("select_kernel", SELECT_KERNEL),
        ("op_quantized_matmul_fused", OP_QMM_FUSED),
        ("linear_describe", LINEAR_DESCRIBE),
        ("linear_load", LINEAR_LOAD),
        ("linear_free", LINEAR_FREE),
        ("_reserved", C.c_void_p * 4),
    ]


QUANT_INIT_FN = C.CFUNCTYPE(C.c_bool, C.POINTER(C.POINTER(QuantVtbl)))


def check_layout() -> None:
    """The same pins the C header asserts (LP64)."""
    assert C.sizeof(BackendVtbl) == 512, C.sizeof(BackendVtbl)
    assert BackendVtbl.op_matmul_f32.offset == 19 * 8
    assert BackendVtbl.op_copy_f32.offset == 38 * 8
    assert BackendVtbl.op_kzg_verify.offset == 59 * 8
    assert BackendVtbl._reserved.offset == 480
    assert C.sizeof(BackendDesc) == 40 and BackendDesc.vtbl.offset == 32
    assert C.sizeof(DeviceInfo) == 48 and DeviceInfo.is_unified_memory.offset == 41
    assert C.sizeof(QuantVtbl) == 8 + 14 * 8 and QuantVtbl.op_quantized_matmul_fused.offset == 8 + 6 * 8
    assert QuantVtbl.linear_free.offset == 80 and C.sizeof(LinearInfo) == 96


check_layout()
