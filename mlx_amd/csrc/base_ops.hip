// base_ops.hip -- the plugin ABI's f32 tensor ops on the GPU: elementwise
// add / sub / mul / div, matmul and transpose, with the reference CPU
// backend's semantics (src/cpu_backend.cpp:185-266): IEEE fp32 per element,
// and for matmul C[M,N] = A[M,K] . B[K,N] (row-major) with every output
// summed in ascending k as a separate multiply and add, so the results are
// bit-identical to the CPU backend's.
#include "kernels.h"

namespace lxq {
namespace {

enum : int { EW_ADD = 0, EW_SUB = 1, EW_MUL = 2, EW_DIV = 3 };

// 4 elements per thread (a 16-byte load of each operand), grid-stride
template <int OP>
__global__ __launch_bounds__(256) void ew_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ o, size_t n) {
#pragma clang fp contract(off)
    const size_t n4 = n / 4;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 x = reinterpret_cast<const float4*>(a)[i], y = reinterpret_cast<const float4*>(b)[i];
        float4 r;
        if constexpr (OP == EW_ADD) r = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
        else if constexpr (OP == EW_SUB) r = make_float4(x.x - y.x, x.y - y.y, x.z - y.z, x.w - y.w);
        else if constexpr (OP == EW_MUL) r = make_float4(x.x * y.x, x.y * y.y, x.z * y.z, x.w * y.w);
        else r = make_float4(x.x / y.x, x.y / y.y, x.z / y.z, x.w / y.w);
        reinterpret_cast<float4*>(o)[i] = r;
    }
    // tail (n % 4 elements) by the first threads
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n - 4 * n4) {
        const size_t i = 4 * n4 + t;
        float r;
        if constexpr (OP == EW_ADD) r = a[i] + b[i];
        else if constexpr (OP == EW_SUB) r = a[i] - b[i];
        else if constexpr (OP == EW_MUL) r = a[i] * b[i];
        else r = a[i] / b[i];
        o[i] = r;
    }
}

// Tiled matmul: a block computes a 64 x 64 tile of C with 256 threads, each a
// 4 x 4 micro-tile; A and B advance through LDS 16 k at a time.  Each
// output's sum still runs k = 0, 1, 2, ... with one rounding per multiply
// and per add (no contraction), the CPU backend's order.
constexpr int TM = 64, TN = 64, TK = 16;

__global__ __launch_bounds__(256) void matmul_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                     float* __restrict__ C, int M, int K, int N) {
#pragma clang fp contract(off)
    __shared__ float As[TK][TM + 4];  // A tile transposed: As[k][m]
    __shared__ float Bs[TK][TN + 4];
    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;  // micro-tile column / row group
    const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += TK) {
        // 1024 elements of each tile, 4 per thread
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int e = tid + 256 * r;
            const int am = e / TK, ak = e % TK;  // A: 64 rows x 16 k
            const int gm = m0 + am, gk = k0 + ak;
            As[ak][am] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.f;
            const int bk = e / TN, bn = e % TN;  // B: 16 k x 64 columns
            const int hk = k0 + bk, hn = n0 + bn;
            Bs[bk][bn] = (hk < K && hn < N) ? B[(size_t)hk * N + hn] : 0.f;
        }
        __syncthreads();
        const int kn = K - k0 < TK ? K - k0 : TK;  // padded k never enters a sum
        for (int k = 0; k < kn; k++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = As[k][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = Bs[k][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + a[i] * b[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
            if (m < M && n < N) C[(size_t)m * N + n] = acc[i][j];
        }
}

// out[c][r] = in[r][c] through a 32 x 33 LDS tile (conflict-free both ways)
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                        int rows, int cols) {
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 32 x 8 threads
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) t[i][tx] = in[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) out[(size_t)c * rows + r] = t[tx][i];
    }
}

}  // namespace

LuxStatus launch_elementwise(int op, const float* a, const float* b, float* o, size_t n, hipStream_t st) {
    if (n == 0) return LuxStatus::Ok;
    size_t blocks = (n / 4 + 255) / 256;
    blocks = blocks < 1 ? 1 : blocks > 65536 ? 65536 : blocks;
    switch (op) {
    case EW_ADD: hipLaunchKernelGGL(ew_kernel<EW_ADD>, dim3((unsigned)blocks), dim3(256), 0, st, a, b, o, n); break;
    case EW_SUB: hipLaunchKernelGGL(ew_kernel<EW_SUB>, dim3((unsigned)blocks), dim3(256), 0, st, a, b, o, n); break;
    case EW_MUL: hipLaunchKernelGGL(ew_kernel<EW_MUL>, dim3((unsigned)blocks), dim3(256), 0, st, a, b, o, n); break;
    case EW_DIV: hipLaunchKernelGGL(ew_kernel<EW_DIV>, dim3((unsigned)blocks), dim3(256), 0, st, a, b, o, n); break;
    default: return LuxStatus::Invalid;
    }
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

LuxStatus launch_matmul_f32(const float* a, const float* b, float* c, int M, int K, int N, hipStream_t st) {
    if (M == 0 || N == 0) return LuxStatus::Ok;
    if (K == 0) return hipMemsetAsync(c, 0, (size_t)M * N * 4, st) == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
    const dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM);
    if (grid.y > 65535) return LuxStatus::NotSupported;
    hipLaunchKernelGGL(matmul_kernel, grid, dim3(256), 0, st, a, b, c, M, K, N);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

LuxStatus launch_transpose_f32(const float* in, float* out, int rows, int cols, hipStream_t st) {
    if (rows == 0 || cols == 0) return LuxStatus::Ok;
    const dim3 grid((cols + 31) / 32, (rows + 31) / 32);
    if (grid.y > 65535) return LuxStatus::NotSupported;
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, st, in, out, rows, cols);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

}  // namespace lxq
