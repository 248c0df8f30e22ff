/* Fake backend plugins for loader tests (CPU only).  Built by the tests with
 *   -DFAKE_NAME='"x"' [-DFAKE_INIT_FALSE] [-DFAKE_ABI=1] [-DFAKE_NULL_CTX]
 *   [-DFAKE_QUANT]
 * Each exports lux_gpu_backend_init like a real plugin and forces one of the
 * loader's failure paths (reference src/plugin_loader.hpp:195-223,
 * src/gpu_core.cpp:187-193).  FAKE_QUANT adds host-memory buffers and the
 * quantized-matmul table with a plain fp32 implementation of the format
 * (f32 activations and scales only), for the core library's tests. */
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include "../../include/lux_gpu_quant_backend.h"

#ifndef FAKE_ABI
#define FAKE_ABI LUX_GPU_BACKEND_ABI_VERSION
#endif

static int g_ctx_token;

static LuxBackendContext* fake_create_context(int device_index) {
    (void)device_index;
#ifdef FAKE_NULL_CTX
    return NULL;
#else
    return (LuxBackendContext*)&g_ctx_token;
#endif
}
static void fake_destroy_context(LuxBackendContext* c) { (void)c; }
static LuxBackendError fake_device_count(int* n) { if (!n) return LUX_BACKEND_ERROR_INVALID_ARGUMENT; *n = 1; return LUX_BACKEND_OK; }

static lux_gpu_backend_vtbl g_vtbl;

#ifdef FAKE_QUANT
typedef struct { unsigned char* p; size_t n; } FakeBuf;
static LuxBackendBuffer* fb_alloc(LuxBackendContext* c, size_t n) {
    (void)c;
    FakeBuf* b = (FakeBuf*)malloc(sizeof(FakeBuf));
    if (!b) return NULL;
    b->p = (unsigned char*)calloc(n ? n : 1, 1);
    b->n = n;
    if (!b->p) { free(b); return NULL; }
    return (LuxBackendBuffer*)b;
}
static LuxBackendBuffer* fb_alloc_data(LuxBackendContext* c, const void* d, size_t n) {
    LuxBackendBuffer* b = fb_alloc(c, n);
    if (b && n) memcpy(((FakeBuf*)b)->p, d, n);
    return b;
}
static void fb_free(LuxBackendContext* c, LuxBackendBuffer* b) {
    (void)c;
    if (b) { free(((FakeBuf*)b)->p); free(b); }
}
static LuxBackendError fb_to_host(LuxBackendContext* c, LuxBackendBuffer* b, void* dst, size_t n) {
    (void)c;
    FakeBuf* f = (FakeBuf*)b;
    memcpy(dst, f->p, n < f->n ? n : f->n);
    return LUX_BACKEND_OK;
}
static LuxBackendError fq_matmul(LuxBackendContext* c, LuxBackendBuffer* x, LuxBackendBuffer* wq,
                                 LuxBackendBuffer* s, LuxBackendBuffer* b, LuxBackendBuffer* y, int M, int K,
                                 int N, int gs, int bits, LuxBackendDtype xd, LuxBackendDtype sd,
                                 LuxBackendDtype od) {
    (void)c;
    if (xd != LUX_DTYPE_FLOAT32 || sd != LUX_DTYPE_FLOAT32 || od != LUX_DTYPE_FLOAT32)
        return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    const float* X = (const float*)((FakeBuf*)x)->p;
    const unsigned* W = (const unsigned*)((FakeBuf*)wq)->p;
    const float* S = (const float*)((FakeBuf*)s)->p;
    const float* B = (const float*)((FakeBuf*)b)->p;
    float* Y = (float*)((FakeBuf*)y)->p;
    const int rw = K * bits / 32, G = K / gs;
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.f;
            for (int k = 0; k < K; k++) {
                const long bit = (long)k * bits;
                unsigned long long pair = W[(long)n * rw + bit / 32];
                if (bit % 32 + bits > 32) pair |= (unsigned long long)W[(long)n * rw + bit / 32 + 1] << 32;
                const unsigned q = (unsigned)(pair >> (bit % 32)) & ((1u << bits) - 1u);
                const float w = fmaf(S[(long)n * G + k / gs], (float)q, B[(long)n * G + k / gs]);
                acc = acc + X[(long)m * K + k] * w;
            }
            Y[(long)m * N + n] = acc;
        }
    return LUX_BACKEND_OK;
}
static lux_gpu_quant_vtbl g_qvtbl;
__attribute__((visibility("default"))) bool lux_gpu_backend_quant_init(const lux_gpu_quant_vtbl** out) {
    g_qvtbl.ext_version = LUX_GPU_QUANT_EXT_VERSION;
    g_qvtbl.struct_size = sizeof(g_qvtbl);
    g_qvtbl.op_quantized_matmul = fq_matmul;
    *out = &g_qvtbl;
    return true;
}
#endif

__attribute__((visibility("default"))) bool lux_gpu_backend_init(lux_gpu_backend_desc* out) {
#ifdef FAKE_INIT_FALSE
    (void)out;
    return false;
#else
    g_vtbl.create_context = fake_create_context;
    g_vtbl.destroy_context = fake_destroy_context;
    g_vtbl.get_device_count = fake_device_count;
#ifdef FAKE_QUANT
    g_vtbl.buffer_alloc = fb_alloc;
    g_vtbl.buffer_alloc_with_data = fb_alloc_data;
    g_vtbl.buffer_free = fb_free;
    g_vtbl.buffer_copy_to_host = fb_to_host;
#endif
    out->abi_version = FAKE_ABI;
    out->backend_name = FAKE_NAME;
    out->backend_version = "0.0.0";
    out->capabilities = 0;
    out->vtbl = &g_vtbl;
    return true;
#endif
}
