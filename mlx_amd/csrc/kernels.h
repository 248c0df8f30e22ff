// kernels.h -- launchers of the gfx950 quantized-matmul kernels.  Host code
// validates arguments and buffer sizes before calling these; the launchers
// only check what their kernels' tiling assumes.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lxq {

enum class LuxStatus : int { Ok = 0, Invalid = 1, OutOfMemory = 2, NotSupported = 3, Internal = 5 };

// Every device buffer handed to these launchers is followed by at least
// kTailPad readable bytes (the plugin allocates them, zero-filled), so a
// kernel may copy an array whose size is not a multiple of 16 bytes in whole
// 16-byte chunks.
constexpr size_t kTailPad = 256;

// Output stage shared by the matmul kernels: y[m, n] = act(acc + bias[n])
// in fp32, then rounded (RNE) to out_dt.  relu(v) = v < 0 ? 0 : v (NaN
// passes), silu(v) = v / (1 + exp(-v)), gelu(v) = v/2 (1 + erf(v / sqrt 2)).
enum : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2, ACT_GELU = 3 };
struct Epilogue {
    const void* bias;  // [N] in bias_dt, or nullptr
    int bias_dt;
    int act;
    int out_dt;
};

struct QmmArgs {
    const void* x;        // [M, K] x_dtype
    const uint32_t* wq;   // [N, K*bits/32]
    const void* scales;   // [N, K/group_size] sb_dtype
    const void* biases;   // [N, K/group_size] sb_dtype
    void* y;              // [M, N] out_dtype
    int M, K, N, group_size, bits;
    int x_dtype, sb_dtype, out_dtype;
    const void* bias = nullptr;  // fused epilogue: per-column bias [N] (bias_dtype) or none
    int bias_dtype = 0;
    int act = ACT_NONE;
    // device workspace a kernel may use for partial sums and counters
    // (counters zero between launches); null/0: kernels that need one are skipped
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // launch number on this workspace: never zero, never repeated for one
    // workspace (the large GEMMs' split tiles meet by it, qsplit.h); 0: no
    // split tiles
    uint32_t epoch = 0;
    // dry run: when set, the launcher that would run stores its kernel's
    // name here (the first one, where rows run in chunks) and launches
    // nothing; no device call is made and no pointer is read
    const char** plan = nullptr;
    Epilogue epi() const { return Epilogue{bias, bias_dtype, act, out_dtype}; }
    // kernels are instantiated with and without the output stage: the plain
    // op runs code with no bias or activation path at all
    bool has_epilogue() const { return bias != nullptr || act != ACT_NONE; }
};

// every launcher, once it has decided to run `kernel`: true for a dry run
// (a.plan set), which records the name and returns without launching
inline bool planned(const QmmArgs& a, const char* kernel) {
    if (a.plan == nullptr) return false;
    if (*a.plan == nullptr) *a.plan = kernel;
    return true;
}

// bandwidth-bound dequant-GEMV (any M; tuned for M <= 8); needs K % 64 == 0
LuxStatus launch_qgemv(const QmmArgs& a, hipStream_t st);
// MFMA kernel for 2 <= M <= 16, 4/8-bit codes, f16/bf16 x; NotSupported
// for other shapes (launch_qgemv tries it first)
LuxStatus launch_qmm_skinny(const QmmArgs& a, hipStream_t st);
// MFMA decode kernel for 2 <= M <= 8, 4-bit codes, f16/bf16 x, K % 1024 == 0,
// K <= 8192; NotSupported otherwise (tried first)
LuxStatus launch_qgemv_dec(const QmmArgs& a, hipStream_t st);
// 4x4x4-MFMA decode kernel (256-byte row segments) for 2 <= M <= 8, 4-bit
// codes, f16/bf16 x, K = 2048, 4096 or 8192; NotSupported otherwise
LuxStatus launch_qgemv_q4(const QmmArgs& a, hipStream_t st);
// MFMA kernel with LDS operand rings for 2 <= M <= 16, 4/8-bit codes,
// f16/bf16 x, K % 1024 == 0; NotSupported otherwise (tried before the above)
LuxStatus launch_qgemv_mid(const QmmArgs& a, hipStream_t st);
// small-M MFMA GEMM (8 < M <= 64, f16/bf16 x, K % 1024 == 0); NotSupported
// otherwise (launch_qgemm tries it first)
LuxStatus launch_qgemm_small(const QmmArgs& a, hipStream_t st);
// split-K small-M MFMA GEMM (8 < M <= 64, f16/bf16 x, K % 128 == 0): x read
// once per 128 columns, the K parts summed through a.ws; NotSupported where
// it does not apply or the workspace is too small (tried before the above)
LuxStatus launch_qgemm_sk(const QmmArgs& a, hipStream_t st);
// workspace bytes launch_qgemm_sk uses for this shape given `cap` bytes
// (0: it needs none or does not apply)
size_t qgemm_sk_workspace(int M, int K, int N, int bits, int x_dtype, size_t cap);
// the workspace every caller of the GEMMs provides (a context's, or the
// allocation-free entry point's static one): the same size everywhere, so
// the same shape takes the same split, and the same result bits.  16 MiB of
// partials: the split-K small-M GEMM's largest split (512 blocks of 32 KiB),
// and the large GEMM's split last round (at most 128 tiles, one K half of
// 128 KiB each).  The first KiB holds tile counters and flags.
constexpr size_t kSplitWorkspaceBytes = (16u << 20) + 4096;
// MFMA GEMM for M > 64 with each wave's W operand dequantized in its own
// registers: 4/8-bit codes, f16/bf16 x, K % 1024 == 0; NotSupported otherwise
LuxStatus launch_qgemm_rw(const QmmArgs& a, hipStream_t st);
// MFMA GEMM for f16/bf16 activations; needs K % 64 == 0
LuxStatus launch_qgemm(const QmmArgs& a, hipStream_t st);
// generic one-thread-per-output kernel for shapes the tiled kernels reject
LuxStatus launch_qmm_generic(const QmmArgs& a, hipStream_t st);

// the plugin ABI's f32 tensor ops (base_ops.hip); op: 0 add, 1 sub, 2 mul, 3 div
LuxStatus launch_elementwise(int op, const float* a, const float* b, float* o, size_t n, hipStream_t st);
// C[M, N] = A[M, K] . B[K, N], row-major, ascending-k sums without contraction
LuxStatus launch_matmul_f32(const float* a, const float* b, float* c, int M, int K, int N, hipStream_t st);
// out[cols, rows] = in[rows, cols]^T
LuxStatus launch_transpose_f32(const float* in, float* out, int rows, int cols, hipStream_t st);

// out[N, K] = dequant(w_q) in out_dtype
LuxStatus launch_dequantize(const uint32_t* wq, const void* scales, const void* biases, void* out,
                            int N, int K, int group_size, int bits, int sb_dtype, int out_dtype,
                            hipStream_t st);
// w[N, K] (w_dtype) -> w_q, scales, biases
LuxStatus launch_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int N, int K,
                          int group_size, int bits, int w_dtype, int sb_dtype, hipStream_t st);

}  // namespace lxq
