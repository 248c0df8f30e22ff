/*
 * lux_gpu_backend_abi.h -- the Lux GPU backend plugin ABI, version 2, as the
 * HIP plugin (libluxgpu_backend_hip.so) implements it.
 *
 * This is a layout-identical restatement of the reference's plugin header
 * (reference include/lux/gpu/backend_plugin.h:24-445): same version number,
 * enum values, struct member order and types, and the same exported init
 * symbol, so a loader built against the reference header loads this plugin
 * unchanged.  Member names are kept so that code written against the
 * reference header compiles against this one.  The static assertions at the
 * end pin the x86-64/LP64 layout (vtable 64 pointer slots = 512 bytes,
 * descriptor 40 bytes, device info 48 bytes).
 */
#ifndef LUX_GPU_BACKEND_ABI_H
#define LUX_GPU_BACKEND_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/lux/gpu/backend_plugin.h:24 (README.md:82 still says 1;
 * the loader compares against this value, src/plugin_loader.hpp:214) */
#define LUX_GPU_BACKEND_ABI_VERSION 2

/* opaque handles (backend_plugin.h:30-32) */
typedef struct LuxBackendContext LuxBackendContext;
typedef struct LuxBackendBuffer LuxBackendBuffer;
typedef struct LuxBackendKernel LuxBackendKernel;

/* element types (backend_plugin.h:38-47); packed quantized weights travel as
 * untyped byte buffers with UINT32 semantics */
typedef enum {
    LUX_DTYPE_FLOAT32 = 0,
    LUX_DTYPE_FLOAT16 = 1,
    LUX_DTYPE_BFLOAT16 = 2,
    LUX_DTYPE_INT32 = 3,
    LUX_DTYPE_INT64 = 4,
    LUX_DTYPE_UINT32 = 5,
    LUX_DTYPE_UINT64 = 6,
    LUX_DTYPE_BOOL = 7,
} LuxBackendDtype;

/* status codes (backend_plugin.h:49-56) */
typedef enum {
    LUX_BACKEND_OK = 0,
    LUX_BACKEND_ERROR_INVALID_ARGUMENT = 1,
    LUX_BACKEND_ERROR_OUT_OF_MEMORY = 2,
    LUX_BACKEND_ERROR_NOT_SUPPORTED = 3,
    LUX_BACKEND_ERROR_DEVICE_LOST = 4,
    LUX_BACKEND_ERROR_INTERNAL = 5,
} LuxBackendError;

/* backend_plugin.h:58-67 */
typedef struct {
    const char* name;
    const char* vendor;
    uint64_t memory_total;
    uint64_t memory_available;
    int compute_units;
    int max_workgroup_size;
    bool is_discrete;
    bool is_unified_memory;
} LuxBackendDeviceInfo;

typedef LuxBackendBuffer Buf_;   /* local shorthand for the slot list below */
typedef LuxBackendContext Ctx_;

/* The 64-slot function table (backend_plugin.h:82-382).  Slot order is the
 * ABI; a backend leaves a slot NULL for "not supported". */
typedef struct lux_gpu_backend_vtbl {
    /* 0-1 lifecycle */
    Ctx_* (*create_context)(int device_index);
    void (*destroy_context)(Ctx_* ctx);
    /* 2-3 device info */
    LuxBackendError (*get_device_count)(int* count);
    LuxBackendError (*get_device_info)(Ctx_* ctx, LuxBackendDeviceInfo* info);
    /* 4 synchronisation */
    LuxBackendError (*sync)(Ctx_* ctx);
    /* 5-10 buffers */
    Buf_* (*buffer_alloc)(Ctx_* ctx, size_t bytes);
    Buf_* (*buffer_alloc_with_data)(Ctx_* ctx, const void* data, size_t bytes);
    void (*buffer_free)(Ctx_* ctx, Buf_* buf);
    LuxBackendError (*buffer_copy_to_host)(Ctx_* ctx, Buf_* buf, void* dst, size_t bytes);
    LuxBackendError (*buffer_copy_from_host)(Ctx_* ctx, Buf_* buf, const void* src, size_t bytes);
    void* (*buffer_get_host_ptr)(Ctx_* ctx, Buf_* buf);
    /* 11-14 custom kernels */
    LuxBackendKernel* (*kernel_load)(Ctx_* ctx, const char* source, const char* entry_point);
    LuxBackendKernel* (*kernel_load_binary)(Ctx_* ctx, const void* binary, size_t size,
                                            const char* entry_point);
    void (*kernel_destroy)(Ctx_* ctx, LuxBackendKernel* kernel);
    LuxBackendError (*kernel_dispatch)(Ctx_* ctx, LuxBackendKernel* kernel,
                                       uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                                       uint32_t block_x, uint32_t block_y, uint32_t block_z,
                                       Buf_** buffers, int num_buffers);
    /* 15-18 elementwise f32 */
    LuxBackendError (*op_add_f32)(Ctx_* ctx, Buf_* a, Buf_* b, Buf_* out, size_t n);
    LuxBackendError (*op_sub_f32)(Ctx_* ctx, Buf_* a, Buf_* b, Buf_* out, size_t n);
    LuxBackendError (*op_mul_f32)(Ctx_* ctx, Buf_* a, Buf_* b, Buf_* out, size_t n);
    LuxBackendError (*op_div_f32)(Ctx_* ctx, Buf_* a, Buf_* b, Buf_* out, size_t n);
    /* 19-20 matrix: C[M,N] = A[M,K] B[K,N], row-major */
    LuxBackendError (*op_matmul_f32)(Ctx_* ctx, Buf_* a, Buf_* b, Buf_* out, int M, int K, int N);
    LuxBackendError (*op_transpose_f32)(Ctx_* ctx, Buf_* in, Buf_* out, int rows, int cols);
    /* 21-26 reductions */
    LuxBackendError (*op_reduce_sum_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_reduce_max_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_reduce_min_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_reduce_mean_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_reduce_sum_axis_f32)(Ctx_* ctx, Buf_* in, Buf_* out,
                                              size_t outer_size, size_t inner_size);
    LuxBackendError (*op_reduce_max_axis_f32)(Ctx_* ctx, Buf_* in, Buf_* out,
                                              size_t outer_size, size_t inner_size);
    /* 27-28 softmax */
    LuxBackendError (*op_softmax_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t batch_size, size_t dim);
    LuxBackendError (*op_log_softmax_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t batch_size,
                                          size_t dim);
    /* 29-37 unary */
    LuxBackendError (*op_exp_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_log_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_sqrt_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_neg_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_abs_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_tanh_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_sigmoid_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_relu_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    LuxBackendError (*op_gelu_f32)(Ctx_* ctx, Buf_* in, Buf_* out, size_t n);
    /* 38 copy */
    LuxBackendError (*op_copy_f32)(Ctx_* ctx, Buf_* src, Buf_* dst, size_t n);
    /* 39-40 normalisation */
    LuxBackendError (*op_layer_norm_f32)(Ctx_* ctx, Buf_* in, Buf_* out, Buf_* gamma, Buf_* beta,
                                         size_t batch_size, size_t dim, float eps);
    LuxBackendError (*op_rms_norm_f32)(Ctx_* ctx, Buf_* in, Buf_* out, Buf_* weight,
                                       size_t batch_size, size_t dim, float eps);
    /* 41-43 NTT / MSM (host pointers) */
    LuxBackendError (*op_ntt_forward)(Ctx_* ctx, uint64_t* data, size_t n, uint64_t modulus);
    LuxBackendError (*op_ntt_inverse)(Ctx_* ctx, uint64_t* data, size_t n, uint64_t modulus);
    LuxBackendError (*op_msm)(Ctx_* ctx, const void* scalars, const void* points, void* result,
                              size_t n, int curve_type);
    /* 44-49 FHE */
    LuxBackendError (*op_poly_mul)(Ctx_* ctx, const uint64_t* a, const uint64_t* b,
                                   uint64_t* result, size_t n, uint64_t modulus);
    LuxBackendError (*op_tfhe_bootstrap)(Ctx_* ctx, const uint64_t* lwe_in, uint64_t* lwe_out,
                                         const uint64_t* bsk, const uint64_t* test_poly,
                                         uint32_t n_lwe, uint32_t N, uint32_t k, uint32_t l,
                                         uint64_t q);
    LuxBackendError (*op_tfhe_keyswitch)(Ctx_* ctx, const uint64_t* lwe_in, uint64_t* lwe_out,
                                         const uint64_t* ksk, uint32_t n_in, uint32_t n_out,
                                         uint32_t l, uint32_t base_log, uint64_t q);
    LuxBackendError (*op_blind_rotate)(Ctx_* ctx, uint64_t* acc, const uint64_t* bsk,
                                       const uint64_t* lwe_a, uint32_t n_lwe, uint32_t N,
                                       uint32_t k, uint32_t l, uint64_t q);
    LuxBackendError (*op_sample_extract)(Ctx_* ctx, const uint64_t* glwe, uint64_t* lwe,
                                         uint32_t N, uint32_t k, uint64_t q);
    LuxBackendError (*op_sample_ntt)(Ctx_* ctx, uint64_t* output, size_t n, uint64_t modulus,
                                     double sigma, uint64_t seed);
    /* 50-51 hashes */
    LuxBackendError (*op_poseidon2_hash)(Ctx_* ctx, const uint64_t* inputs, uint64_t* outputs,
                                         size_t rate, size_t num_hashes);
    LuxBackendError (*op_blake3_hash)(Ctx_* ctx, const uint8_t* inputs, uint8_t* outputs,
                                      const size_t* input_lens, size_t num_hashes);
    /* 52-56 curves */
    LuxBackendError (*op_bls12_381_add)(Ctx_* ctx, const void* a, const void* b, void* out,
                                        size_t n, bool is_g2);
    LuxBackendError (*op_bls12_381_mul)(Ctx_* ctx, const void* points, const void* scalars,
                                        void* out, size_t n, bool is_g2);
    LuxBackendError (*op_bls12_381_pairing)(Ctx_* ctx, const void* g1_points,
                                            const void* g2_points, void* out, size_t n);
    LuxBackendError (*op_bn254_add)(Ctx_* ctx, const void* a, const void* b, void* out, size_t n,
                                    bool is_g2);
    LuxBackendError (*op_bn254_mul)(Ctx_* ctx, const void* points, const void* scalars, void* out,
                                    size_t n, bool is_g2);
    /* 57-59 KZG */
    LuxBackendError (*op_kzg_commit)(Ctx_* ctx, const void* coeffs, const void* srs,
                                     void* commitment, size_t degree, int curve_type);
    LuxBackendError (*op_kzg_open)(Ctx_* ctx, const void* coeffs, const void* srs,
                                   const void* point, void* proof, size_t degree, int curve_type);
    LuxBackendError (*op_kzg_verify)(Ctx_* ctx, const void* commitment, const void* proof,
                                     const void* point, const void* value, const void* srs_g2,
                                     bool* result, int curve_type);
    /* 60-63 reserved */
    void* _reserved[4];
} lux_gpu_backend_vtbl;

/* descriptor filled by the init symbol (backend_plugin.h:388-394); the
 * loader keeps the string and vtable pointers, so they must be static */
typedef struct {
    uint32_t abi_version;
    const char* backend_name;
    const char* backend_version;
    uint32_t capabilities;
    const lux_gpu_backend_vtbl* vtbl;
} lux_gpu_backend_desc;

/* capability bits (backend_plugin.h:397-415) */
#define LUX_CAP_TENSOR_OPS     (1u << 0)
#define LUX_CAP_MATMUL         (1u << 1)
#define LUX_CAP_NTT            (1u << 2)
#define LUX_CAP_MSM            (1u << 3)
#define LUX_CAP_CUSTOM_KERNELS (1u << 4)
#define LUX_CAP_UNIFIED_MEMORY (1u << 5)
#define LUX_CAP_FHE            (1u << 6)
#define LUX_CAP_TFHE           (1u << 7)
#define LUX_CAP_REDUCE         (1u << 8)
#define LUX_CAP_SOFTMAX        (1u << 9)
#define LUX_CAP_UNARY          (1u << 10)
#define LUX_CAP_NORMALIZATION  (1u << 11)
#define LUX_CAP_BLS12_381      (1u << 12)
#define LUX_CAP_BN254          (1u << 13)
#define LUX_CAP_KZG            (1u << 14)
#define LUX_CAP_POSEIDON2      (1u << 15)
#define LUX_CAP_BLAKE3         (1u << 16)
#define LUX_CAP_BLIND_ROTATE   (1u << 17)
#define LUX_CAP_POLY_MUL       (1u << 18)

/* entry point (backend_plugin.h:421-426) */
typedef bool (*lux_gpu_backend_init_fn)(lux_gpu_backend_desc* out);
#define LUX_GPU_BACKEND_INIT_SYMBOL "lux_gpu_backend_init"

/*
 * Exported by libluxgpu_backend_hip.so.  Replaces, for the name "hip", what
 * the reference loader dlsym()s from libluxgpu_backend_<name>.so
 * (reference src/plugin_loader.hpp:165-209).  Fills *out and returns true
 * when at least one gfx950 device is present; returns false (backend
 * unavailable, reference src/plugin_loader.hpp:209-211) otherwise.
 */
__attribute__((visibility("default"))) bool lux_gpu_backend_init(lux_gpu_backend_desc* out);

#ifdef __cplusplus
}
#endif

/* layout pins: LP64 (x86-64 / aarch64 Linux) */
#if defined(__LP64__)
#ifdef __cplusplus
#define LUX_ABI_ASSERT(c, m) static_assert(c, m)
#else
#define LUX_ABI_ASSERT(c, m) _Static_assert(c, m)
#endif
LUX_ABI_ASSERT(sizeof(lux_gpu_backend_vtbl) == 512, "vtable must be 64 pointer slots");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_vtbl, op_matmul_f32) == 19 * 8, "op_matmul_f32 slot");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_vtbl, op_copy_f32) == 38 * 8, "op_copy_f32 slot");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_vtbl, op_ntt_forward) == 41 * 8, "op_ntt_forward slot");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_vtbl, op_kzg_verify) == 59 * 8, "op_kzg_verify slot");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_vtbl, _reserved) == 480, "reserved slots");
LUX_ABI_ASSERT(sizeof(lux_gpu_backend_desc) == 40, "descriptor size");
LUX_ABI_ASSERT(offsetof(lux_gpu_backend_desc, vtbl) == 32, "descriptor vtbl offset");
LUX_ABI_ASSERT(sizeof(LuxBackendDeviceInfo) == 48, "device info size");
LUX_ABI_ASSERT(offsetof(LuxBackendDeviceInfo, is_unified_memory) == 41, "device info flags");
LUX_ABI_ASSERT(sizeof(LuxBackendError) == 4 && sizeof(LuxBackendDtype) == 4, "enum size");
#undef LUX_ABI_ASSERT
#endif

#endif /* LUX_GPU_BACKEND_ABI_H */
