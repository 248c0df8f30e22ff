/* Prints the byte offset of every vtable slot, then the descriptor and device
 * info layout, one number per line.  Compiled once against this project's
 * header and once against the reference's (-DUSE_REF) by the ABI tests. */
#include <stddef.h>
#include <stdio.h>
#ifdef USE_REF
#include "lux/gpu/backend_plugin.h"
#else
#include "../../include/lux_gpu_backend_abi.h"
#endif

#define S(m) printf("%zu\n", offsetof(lux_gpu_backend_vtbl, m))
int main(void) {
    S(create_context); S(destroy_context); S(get_device_count); S(get_device_info); S(sync);
    S(buffer_alloc); S(buffer_alloc_with_data); S(buffer_free); S(buffer_copy_to_host);
    S(buffer_copy_from_host); S(buffer_get_host_ptr); S(kernel_load); S(kernel_load_binary);
    S(kernel_destroy); S(kernel_dispatch); S(op_add_f32); S(op_sub_f32); S(op_mul_f32);
    S(op_div_f32); S(op_matmul_f32); S(op_transpose_f32); S(op_reduce_sum_f32);
    S(op_reduce_max_f32); S(op_reduce_min_f32); S(op_reduce_mean_f32); S(op_reduce_sum_axis_f32);
    S(op_reduce_max_axis_f32); S(op_softmax_f32); S(op_log_softmax_f32); S(op_exp_f32);
    S(op_log_f32); S(op_sqrt_f32); S(op_neg_f32); S(op_abs_f32); S(op_tanh_f32);
    S(op_sigmoid_f32); S(op_relu_f32); S(op_gelu_f32); S(op_copy_f32); S(op_layer_norm_f32);
    S(op_rms_norm_f32); S(op_ntt_forward); S(op_ntt_inverse); S(op_msm); S(op_poly_mul);
    S(op_tfhe_bootstrap); S(op_tfhe_keyswitch); S(op_blind_rotate); S(op_sample_extract);
    S(op_sample_ntt); S(op_poseidon2_hash); S(op_blake3_hash); S(op_bls12_381_add);
    S(op_bls12_381_mul); S(op_bls12_381_pairing); S(op_bn254_add); S(op_bn254_mul);
    S(op_kzg_commit); S(op_kzg_open); S(op_kzg_verify); S(_reserved);
    printf("%zu\n%zu\n%zu\n%zu\n", sizeof(lux_gpu_backend_vtbl), sizeof(lux_gpu_backend_desc),
           offsetof(lux_gpu_backend_desc, vtbl), sizeof(LuxBackendDeviceInfo));
    printf("%d\n", LUX_GPU_BACKEND_ABI_VERSION);
    return 0;
}
