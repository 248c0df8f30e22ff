/* Fake backend plugins for loader tests (CPU only).  Built by the tests with
 *   -DFAKE_NAME='"x"' [-DFAKE_INIT_FALSE] [-DFAKE_ABI=1] [-DFAKE_NULL_CTX]
 * Each exports lux_gpu_backend_init like a real plugin and forces one of the
 * loader's failure paths (reference src/plugin_loader.hpp:195-223,
 * src/gpu_core.cpp:187-193). */
#include <stdlib.h>
#include "../../include/lux_gpu_backend_abi.h"

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

__attribute__((visibility("default"))) bool lux_gpu_backend_init(lux_gpu_backend_desc* out) {
#ifdef FAKE_INIT_FALSE
    (void)out;
    return false;
#else
    g_vtbl.create_context = fake_create_context;
    g_vtbl.destroy_context = fake_destroy_context;
    g_vtbl.get_device_count = fake_device_count;
    out->abi_version = FAKE_ABI;
    out->backend_name = FAKE_NAME;
    out->backend_version = "0.0.0";
    out->capabilities = 0;
    out->vtbl = &g_vtbl;
    return true;
#endif
}
