// qgemm_sk.hip -- dispatch of the split-K small-M GEMM (kernel in qgemm_sk.h,
// one translation unit per code width: qgemm_sk_b{2,3,4,5,6,8}.hip).
#include "qgemm_sk.h"

namespace lxq {
namespace sk {

extern template LuxStatus launch_bits<2>(const QmmArgs&, int, hipStream_t);
extern template LuxStatus launch_bits<3>(const QmmArgs&, int, hipStream_t);
extern template LuxStatus launch_bits<4>(const QmmArgs&, int, hipStream_t);
extern template LuxStatus launch_bits<5>(const QmmArgs&, int, hipStream_t);
extern template LuxStatus launch_bits<6>(const QmmArgs&, int, hipStream_t);
extern template LuxStatus launch_bits<8>(const QmmArgs&, int, hipStream_t);

// Measured (K = 4096, 4-bit g64 f16, weights streamed from HBM: eight
// copies in rotation; µs per launch against the W-streaming kernel):
// unsplit, with x read once per 128 columns, this kernel wins on wide N
// (N = 28672 / 32768: M = 64 38.4 / 39.7 against 47.5 / 50.1, M = 32 32.1
// against 37.8, M = 16 31.5 against 37.1); split, the partial sums and the
// last part's fixup add 5-8 µs, and on narrower N it loses (N = 11008
// 3-bit M = 64: 26.2 at best, S = 2, against 23.6; N = 14336 M = 64 26.4
// against 22.9).  So it runs unsplit from kUnsplitTiles tiles on, and split
// only where the W-streaming kernel does not apply (K % 1024 != 0).
constexpr int kUnsplitTiles = 192;
// at most two blocks per CU; this also bounds the partials: 512 blocks x
// 32 KiB = 16 MiB
constexpr int kMaxBlocks = 512;

bool applies(int M, int K, int N, int bits, int x_dtype) {
    if (M <= 8 || M > 64 || N <= 0 || (x_dtype != DT_F16 && x_dtype != DT_BF16) || K % kSS != 0) return false;
    if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8) return false;
    // buffer offsets are 32-bit
    if ((size_t)M * K * 2 >= (1ull << 31) || (size_t)N * K * bits / 8 >= (1ull << 31) ||
        (size_t)N * (K / 32) * 4 >= (1ull << 31))
        return false;
    // narrow N with K % 1024 == 0: the W-streaming kernel is faster
    return (N + kCols - 1) / kCols >= kUnsplitTiles || K % 1024 != 0;
}

// the number of K parts S: 1 from kUnsplitTiles tiles on; else a divisor of
// K / 128 leaving at least 2 super-steps per part, the smallest that gives
// kUnsplitTiles blocks without passing kMaxBlocks (else the largest below
// kMaxBlocks), lowered until the workspace fits `cap`
int choose_split(int M, int K, int N, size_t cap) {
    static_assert(kUnsplitTiles <= kMaxSplitTiles, "split tiles have counter slots");
    const int tiles = (N + kCols - 1) / kCols, steps = K / kSS;
    if (tiles >= kUnsplitTiles) return 1;
    int S = 1;
    for (int d = 2; d <= steps / 2; d++) {
        if (steps % d != 0) continue;
        if (tiles * d > kMaxBlocks) break;
        S = d;
        if (tiles * d >= kUnsplitTiles) break;
    }
    while (S > 1 && ws_bytes(S, M, N) > cap) {
        int d = S - 1;
        while (d > 1 && steps % d != 0) d--;
        S = d;
    }
    return S;
}

}  // namespace sk

size_t qgemm_sk_workspace(int M, int K, int N, int bits, int x_dtype, size_t cap) {
    using namespace sk;
    if (!applies(M, K, N, bits, x_dtype)) return 0;
    const int S = choose_split(M, K, N, cap);
    return S > 1 ? ws_bytes(S, M, N) : 0;
}

LuxStatus launch_qgemm_sk(const QmmArgs& a, hipStream_t st) {
    using namespace sk;
    if (!applies(a.M, a.K, a.N, a.bits, a.x_dtype)) return LuxStatus::NotSupported;
    const size_t cap = a.ws ? a.ws_bytes : 0;
    const int S = choose_split(a.M, a.K, a.N, cap);
    // what the kernel writes when it splits: partials within the workspace,
    // one counter slot per tile
    if (S > 1 && (ws_bytes(S, a.M, a.N) > cap || (a.N + kCols - 1) / kCols > kMaxSplitTiles))
        return LuxStatus::Internal;
    switch (a.bits) {
    case 2: return launch_bits<2>(a, S, st);
    case 3: return launch_bits<3>(a, S, st);
    case 4: return launch_bits<4>(a, S, st);
    case 5: return launch_bits<5>(a, S, st);
    case 6: return launch_bits<6>(a, S, st);
    default: return launch_bits<8>(a, S, st);
    }
}

}  // namespace lxq
