// ref_loader_probe.cpp -- drives the REFERENCE's own plugin loader
// (reference src/plugin_loader.hpp, compiled from its header where it lies)
// against a plugin library, and reports what it did as one JSON line.
//
//   ref_loader_probe <name>      load_backend(<name>) via LUX_GPU_BACKEND_PATH
//   ref_loader_probe --path <p>  load_backend_from_path(<p>)
//
// When the backend is available it also runs the reference's dense-matmul
// known answer through the quant extension: [[1,2],[3,4]] x [[5,6],[7,8]]
// = [[19,22],[43,50]] (reference test/test_core.cpp:95-117), expressed as a
// 4-bit quantized matmul with scale 1 and bias 0 (codes are the integers).
// Test infrastructure only.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include <dlfcn.h>  // before the reference header, which includes it inside its namespace

#include "plugin_loader.hpp"

typedef int (*qmm_fn)(LuxBackendContext*, LuxBackendBuffer*, LuxBackendBuffer*, LuxBackendBuffer*,
                      LuxBackendBuffer*, LuxBackendBuffer*, int, int, int, int, int, int, int, int);

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <name> | --path <lib>\n", argv[0]);
        return 2;
    }
    auto& L = lux::gpu::PluginLoader::instance();
    bool ok;
    std::string name;
    if (std::strcmp(argv[1], "--path") == 0 && argc > 2) {
        ok = L.load_backend_from_path(argv[2]);
        name = "hip";
    } else {
        name = argv[1];
        ok = L.load_backend(name);
    }
    const lux::gpu::LoadedBackend* b = L.get_backend(name);
    std::printf("{\"loaded\": %s, \"available\": %s", ok ? "true" : "false", b ? "true" : "false");
    if (!b) {
        std::printf("}\n");
        return 0;
    }
    std::printf(", \"abi_version\": %u, \"backend_name\": \"%s\", \"capabilities\": %u",
                b->desc.abi_version, b->desc.backend_name, b->desc.capabilities);
    const lux_gpu_backend_vtbl* v = b->desc.vtbl;
    LuxBackendContext* ctx = v->create_context(0);
    std::printf(", \"context\": %s", ctx ? "true" : "false");
    // the quant extension: looked up next to the init symbol
    typedef bool (*qinit_fn)(const void**);
    qinit_fn qinit = reinterpret_cast<qinit_fn>(dlsym(b->handle, "lux_gpu_backend_quant_init"));
    const void* qt = nullptr;
    if (ctx && qinit && qinit(&qt) && qt) {
        // ext_version, struct_size, then op_quantized_matmul
        const uint32_t* hdr = static_cast<const uint32_t*>(qt);
        qmm_fn qmm = *reinterpret_cast<const qmm_fn*>(static_cast<const char*>(qt) + 8);
        const int M = 2, K = 64, N = 2;
        float x[M * K] = {0};
        x[0] = 1; x[1] = 2; x[K] = 3; x[K + 1] = 4;
        uint32_t wq[N * K / 8] = {0};
        wq[0] = 5u | (7u << 4);              // row n=0: B[:,0] = (5, 7)
        wq[K / 8] = 6u | (8u << 4);          // row n=1: B[:,1] = (6, 8)
        float s[N] = {1.f, 1.f}, bias[N] = {0.f, 0.f}, y[M * N] = {0};
        LuxBackendBuffer* bx = v->buffer_alloc_with_data(ctx, x, sizeof(x));
        LuxBackendBuffer* bw = v->buffer_alloc_with_data(ctx, wq, sizeof(wq));
        LuxBackendBuffer* bs = v->buffer_alloc_with_data(ctx, s, sizeof(s));
        LuxBackendBuffer* bb = v->buffer_alloc_with_data(ctx, bias, sizeof(bias));
        LuxBackendBuffer* by = v->buffer_alloc(ctx, sizeof(y));
        int rc = qmm(ctx, bx, bw, bs, bb, by, M, K, N, 64, 4, LUX_DTYPE_FLOAT32, LUX_DTYPE_FLOAT32,
                     LUX_DTYPE_FLOAT32);
        int rc2 = v->buffer_copy_to_host(ctx, by, y, sizeof(y));
        std::printf(", \"quant_ext_version\": %u, \"qmm_rc\": %d, \"copy_rc\": %d, "
                    "\"y\": [%g, %g, %g, %g]",
                    hdr[0], rc, rc2, y[0], y[1], y[2], y[3]);
        for (LuxBackendBuffer* p : {bx, bw, bs, bb, by}) v->buffer_free(ctx, p);
    }
    if (ctx) v->destroy_context(ctx);
    std::printf("}\n");
    return 0;
}
