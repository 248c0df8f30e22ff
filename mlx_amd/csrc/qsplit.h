// qsplit.h -- the split-work workspace of the GEMMs: its layout, and the
// protocol by which the two K halves of a large-GEMM tile meet.
//
// Every caller of the GEMMs provides one workspace of kSplitWorkspaceBytes
// (a context's buffer, zero-filled at allocation, or the allocation-free
// entry point's static array, cleared once).  Layout:
//   bytes [0, 1024)      split-K small-M GEMM tile counters (256 words; that
//                        kernel returns each to zero at the end of a launch)
//   bytes [1024, 1536)   large-GEMM split-tile arrival counters (128 words)
//   bytes [1536, 2048)   large-GEMM split-tile flags (128 words)
//   bytes [2048, 3072)   register-W GEMM K-part counters (256 words; the
//                        last part of a tile returns its counter to zero)
//   bytes [4096, ...)    partial sums of whichever kernel runs (meaningful
//                        only within the launch that writes them)
// The two kernels' words never overlap, so neither can disturb the other's
// counts, whatever a launch leaves behind.
//
// Split tile protocol (large GEMMs).  Each half counts in on the tile's
// counter once its fp32 sums are final.  The counter only ever grows by two
// per launch and starts even, so the first half to arrive reads an even
// count: it stores its sums to the workspace and then raises the tile's
// flag to this launch's epoch (a per-workspace launch number the host
// passes, never zero and never repeated for a workspace).  The second reads
// an odd count: its partner has already counted in -- it is resident and
// past its K loop -- so it waits for the flag to equal the epoch, adds the
// stored sums to its own (one fp32 addition per value, the same whichever
// half is first) and stores y.  Nothing is reset: a flag from an earlier
// launch holds an older epoch and never satisfies a later wait, and a wait
// that gives up (a bounded number of polls) leaves the counts consistent for
// the next launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lxq {
namespace split {

constexpr size_t kSkCounterBytes = 1024;
constexpr int kHalfCounterWord = 256;
constexpr int kHalfFlagWord = 384;
constexpr int kMaxHalfTiles = 128;
constexpr int kPartCounterWord = 512;
constexpr int kMaxPartTiles = 256;
constexpr size_t kPartOffset = 4096;
// cache policy of the workspace accesses: device scope (sc1).  The halves
// may run on different XCDs, whose L2s are not coherent with each other.
constexpr int kCachePolicyDevice = 16;
static_assert(kHalfFlagWord + kMaxHalfTiles <= (int)(kPartOffset / 4), "split words below the partial sums");
static_assert(kSkCounterBytes <= (size_t)kHalfCounterWord * 4, "split-K counters below the large-GEMM words");

static_assert(kHalfFlagWord + kMaxHalfTiles <= kPartCounterWord &&
                  (size_t)(kPartCounterWord + kMaxPartTiles) * 4 <= kPartOffset,
              "K-part counters between the flags and the partial sums");

// K parts (register-W GEMM): one thread per block, after the block's sums
// are stored (vmcnt(0)) and the block has met at a barrier.  true for the
// last of the tile's `parts` to count in, which also sets the counter back
// to zero for the next launch (every other part has counted in by then).
__device__ __forceinline__ bool count_part(void* ws, int tile, int parts) {
    uint32_t* c = static_cast<uint32_t*>(ws) + kPartCounterWord + tile;
    const bool last = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(parts - 1);
    if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// One thread per block.  true: this block is the first of the tile's two
// halves to arrive (it stores its sums, then publish()es); false: the
// second (it waits, then adds).
__device__ __forceinline__ bool arrive_first(void* ws, int st) {
    uint32_t* c = static_cast<uint32_t*>(ws) + kHalfCounterWord + st;
    return (__hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 1u) == 0u;
}

// One thread, after every thread's partial-sum stores have completed
// (vmcnt(0)) and the block has met at a barrier.
__device__ __forceinline__ void publish(void* ws, int st, uint32_t epoch) {
    uint32_t* f = static_cast<uint32_t*>(ws) + kHalfFlagWord + st;
    __hip_atomic_store(f, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One thread: wait (s_sleep between polls, at most 2^22 polls, ~0.3 s)
// for the first half's flag; false if it never came.
__device__ __forceinline__ bool wait_partner(void* ws, int st, uint32_t epoch) {
    const uint32_t* f = static_cast<const uint32_t*>(ws) + kHalfFlagWord + st;
    uint32_t polls = 0;
    while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) {
        if (++polls >= (1u << 22)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    return true;
}

}  // namespace split
}  // namespace lxq
