// lux_quant_core.cpp -- backend selection and the public quantized-matmul op
// (libluxgpu_quant_core.so).  Host code; the behaviour is documented in
// include/lux_quant_core.h.
#include "../../../include/lux_quant_core.h"

#include <dlfcn.h>
#include <sys/stat.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

struct lux_qcore {
    void* handle = nullptr;
    lux_gpu_backend_desc desc{};
    const lux_gpu_quant_vtbl* quant = nullptr;
    LuxBackendContext* ctx = nullptr;
    std::string name;
};

struct lux_qtensor {
    LuxBackendBuffer* buf = nullptr;
    int64_t rows = 0, cols = 0;
    int dtype = 0;
    size_t bytes = 0;
};

namespace {

const char* const kPriority[] = {"metal", "cuda", "hip", "webgpu"};

size_t elem_bytes(int dt) {
    switch (dt) {
    case LUX_DTYPE_FLOAT32: return 4;
    case LUX_DTYPE_FLOAT16: return 2;
    case LUX_DTYPE_BFLOAT16: return 2;
    case LUX_QTENSOR_U32: return 4;
    default: return 0;
    }
}
bool float_dtype(int dt) {
    return dt == LUX_DTYPE_FLOAT32 || dt == LUX_DTYPE_FLOAT16 || dt == LUX_DTYPE_BFLOAT16;
}

bool file_exists(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// the reference's search order plus the directory of this library
std::vector<std::string> search_paths() {
    std::vector<std::string> paths = {"/usr/lib/lux-gpu", "/usr/local/lib/lux-gpu"};
    Dl_info info;
    if (dladdr(reinterpret_cast<const void*>(&lux_qcore_open), &info) && info.dli_fname) {
        std::string self(info.dli_fname);
        const size_t slash = self.rfind('/');
        if (slash != std::string::npos) paths.push_back(self.substr(0, slash));
    }
    if (const char* env = std::getenv("LUX_GPU_BACKEND_PATH")) {
        // each entry is inserted at the front, so the last one is searched first
        std::string s(env);
        size_t start = 0;
        for (;;) {
            const size_t colon = s.find(':', start);
            const std::string part = s.substr(start, colon == std::string::npos ? std::string::npos : colon - start);
            if (!part.empty()) paths.insert(paths.begin(), part);
            if (colon == std::string::npos) break;
            start = colon + 1;
        }
    }
    return paths;
}

// dlopen, init, ABI check and the quantized table; 0 on success, else a message
const char* load_from_path(const std::string& path, lux_qcore& c) {
    void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) return "dlopen failed";
    auto init = reinterpret_cast<lux_gpu_backend_init_fn>(dlsym(h, LUX_GPU_BACKEND_INIT_SYMBOL));
    if (!init) {
        dlclose(h);
        return "no lux_gpu_backend_init";
    }
    lux_gpu_backend_desc d;
    std::memset(&d, 0, sizeof(d));
    if (!init(&d)) {
        dlclose(h);
        return "backend unavailable";
    }
    if (d.abi_version != LUX_GPU_BACKEND_ABI_VERSION) {
        std::fprintf(stderr, "lux-gpu: backend %s has ABI version %u, expected %u\n", path.c_str(), d.abi_version,
                     (unsigned)LUX_GPU_BACKEND_ABI_VERSION);
        dlclose(h);
        return "ABI version mismatch";
    }
    auto qinit = reinterpret_cast<lux_gpu_backend_quant_init_fn>(dlsym(h, LUX_GPU_QUANT_INIT_SYMBOL));
    const lux_gpu_quant_vtbl* q = nullptr;
    if (!qinit || !qinit(&q) || !q || q->ext_version != LUX_GPU_QUANT_EXT_VERSION || !q->op_quantized_matmul) {
        dlclose(h);
        return "backend has no quantized-matmul extension";
    }
    c.handle = h;
    c.desc = d;
    c.quant = q;
    c.name = d.backend_name ? d.backend_name : "";
    return nullptr;
}

// libluxgpu_backend_<name>.so in the first search path that has it
const char* load_named(const std::string& name, lux_qcore& c) {
    for (const auto& d : search_paths()) {
        const std::string p = d + "/libluxgpu_backend_" + name + ".so";
        if (file_exists(p)) return load_from_path(p, c);
    }
    return "backend not found";
}

}  // namespace

extern "C" {

lux_qcore* lux_qcore_open(const char* name, int device, const char** err) {
    const char* dummy;
    if (!err) err = &dummy;
    *err = nullptr;
    std::string want = name ? name : "auto";
    if (want == "auto") {
        const char* env = std::getenv("LUX_BACKEND");
        if (env && *env) want = env;
    }
    for (auto& ch : want) ch = (char)std::tolower((unsigned char)ch);
    if (want.empty()) want = "auto";
    if (want == "cpu") {
        *err = "LUX_BACKEND=cpu selects the core's own CPU backend";
        return nullptr;
    }
    lux_qcore* c = new (std::nothrow) lux_qcore();
    if (!c) {
        *err = "out of memory";
        return nullptr;
    }
    const char* msg = "no backend available";
    if (want == "auto") {
        for (const char* n : kPriority) {
            msg = load_named(n, *c);
            if (!msg) break;
        }
        if (msg) msg = "no backend available";
    } else {
        msg = load_named(want, *c);
    }
    if (!msg) {
        c->ctx = c->desc.vtbl && c->desc.vtbl->create_context ? c->desc.vtbl->create_context(device) : nullptr;
        if (!c->ctx) msg = "create_context failed";
    }
    if (msg) {
        *err = msg;
        lux_qcore_close(c);
        return nullptr;
    }
    return c;
}

void lux_qcore_close(lux_qcore* c) {
    if (!c) return;
    if (c->ctx && c->desc.vtbl && c->desc.vtbl->destroy_context) c->desc.vtbl->destroy_context(c->ctx);
    // the plugin stays loaded until process exit, as the reference loader's
    // static registry keeps it (reference src/plugin_loader.hpp:46-66)
    delete c;
}

const char* lux_qcore_backend_name(const lux_qcore* c) { return c ? c->name.c_str() : nullptr; }
const lux_gpu_backend_vtbl* lux_qcore_vtbl(const lux_qcore* c) { return c ? c->desc.vtbl : nullptr; }
const lux_gpu_quant_vtbl* lux_qcore_quant(const lux_qcore* c) { return c ? c->quant : nullptr; }
LuxBackendContext* lux_qcore_context(const lux_qcore* c) { return c ? c->ctx : nullptr; }

lux_qtensor* lux_qtensor_create(lux_qcore* c, const void* data, int64_t rows, int64_t cols, int dtype) {
    const size_t es = elem_bytes(dtype);
    if (!c || !c->ctx || es == 0 || rows < 0 || cols < 0) return nullptr;
    if (cols && (uint64_t)rows > SIZE_MAX / es / (uint64_t)cols) return nullptr;
    const size_t bytes = (size_t)rows * (size_t)cols * es;
    const lux_gpu_backend_vtbl* v = c->desc.vtbl;
    LuxBackendBuffer* b = nullptr;
    if (data && bytes) b = v->buffer_alloc_with_data ? v->buffer_alloc_with_data(c->ctx, data, bytes) : nullptr;
    else b = v->buffer_alloc ? v->buffer_alloc(c->ctx, bytes ? bytes : 1) : nullptr;
    if (!b) return nullptr;
    lux_qtensor* t = new (std::nothrow) lux_qtensor();
    if (!t) {
        v->buffer_free(c->ctx, b);
        return nullptr;
    }
    t->buf = b;
    t->rows = rows;
    t->cols = cols;
    t->dtype = dtype;
    t->bytes = bytes;
    return t;
}

LuxBackendError lux_qtensor_to_host(lux_qcore* c, const lux_qtensor* t, void* dst, size_t bytes) {
    if (!c || !t || !dst || !c->desc.vtbl->buffer_copy_to_host) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const size_t n = bytes < t->bytes ? bytes : t->bytes;
    if (!n) return LUX_BACKEND_OK;
    return c->desc.vtbl->buffer_copy_to_host(c->ctx, t->buf, dst, n);
}

void lux_qtensor_free(lux_qcore* c, lux_qtensor* t) {
    if (!t) return;
    if (c && c->desc.vtbl && c->desc.vtbl->buffer_free) c->desc.vtbl->buffer_free(c->ctx, t->buf);
    delete t;
}

int64_t lux_qtensor_dim(const lux_qtensor* t, int i) { return !t ? -1 : i == 0 ? t->rows : i == 1 ? t->cols : -1; }
int lux_qtensor_dtype(const lux_qtensor* t) { return t ? t->dtype : -1; }

lux_qtensor* lux_tensor_quantized_matmul(lux_qcore* c, const lux_qtensor* x, const lux_qtensor* w_q,
                                         const lux_qtensor* scales, const lux_qtensor* biases, int group_size,
                                         int bits, LuxBackendError* err_code) {
    LuxBackendError dummy;
    if (!err_code) err_code = &dummy;
    *err_code = LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (!c || !c->quant || !x || !w_q || !scales || !biases || group_size <= 0 || bits <= 0) return nullptr;
    // x [M, K]; w_q [N, K*bits/32] packed; scales = biases [N, K/group_size]
    if (!float_dtype(x->dtype) || w_q->dtype != LUX_QTENSOR_U32 || !float_dtype(scales->dtype) ||
        scales->dtype != biases->dtype)
        return nullptr;
    const int64_t M = x->rows, K = x->cols, N = w_q->rows;
    if (K % group_size || (K * bits) % 32 || w_q->cols != K * bits / 32 || scales->rows != N ||
        scales->cols != K / group_size || biases->rows != N || biases->cols != scales->cols)
        return nullptr;
    if (M > INT32_MAX || K > INT32_MAX || N > INT32_MAX) return nullptr;
    lux_qtensor* y = lux_qtensor_create(c, nullptr, M, N, x->dtype);
    if (!y) {
        *err_code = LUX_BACKEND_ERROR_OUT_OF_MEMORY;
        return nullptr;
    }
    *err_code = c->quant->op_quantized_matmul(c->ctx, x->buf, w_q->buf, scales->buf, biases->buf, y->buf, (int)M,
                                              (int)K, (int)N, group_size, bits, (LuxBackendDtype)x->dtype,
                                              (LuxBackendDtype)scales->dtype, (LuxBackendDtype)x->dtype);
    if (*err_code != LUX_BACKEND_OK) {
        lux_qtensor_free(c, y);
        return nullptr;
    }
    return y;
}

}  // extern "C"
