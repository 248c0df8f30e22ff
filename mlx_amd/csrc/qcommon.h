// qcommon.h -- device helpers shared by the quantized-matmul kernels (gfx950).
//
// Format: row n of W holds K codes of BITS bits in a little-endian bitstream
// of uint32 words (code k at bits [k*BITS, k*BITS+BITS)); scales/biases are
// [N, K/group] in f32/f16/bf16; w_hat = fmaf(scale, q, bias).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace lxq {

enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// round-to-nearest-even conversions (hardware v_cvt_f16_f32 / v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint16_t f32_to_f16(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
}

// value of v after a round trip through dtype dt
__device__ __forceinline__ float round_dt(float v, int dt) {
    if (dt == DT_F32) return v;
    return dt == DT_F16 ? f16_to_f32(f32_to_f16(v)) : bf16_to_f32(f32_to_bf16(v));
}

__device__ __forceinline__ float load_f(const void* p, size_t i, int dt) {
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
    return dt == DT_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}

__device__ __forceinline__ void store_f(void* p, size_t i, int dt, float v) {
    if (dt == DT_F32) reinterpret_cast<float*>(p)[i] = v;
    else if (dt == DT_F16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16(v);
    else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// the output stage (Epilogue, kernels.h) for column n, then the store
__device__ __forceinline__ float apply_epilogue(const Epilogue& e, size_t n, float v) {
    if (e.bias) v = v + load_f(e.bias, n, e.bias_dt);
    if (e.act == ACT_RELU) v = v < 0.f ? 0.f : v;
    else if (e.act == ACT_SILU) v = v / (1.f + expf(-v));
    else if (e.act == ACT_GELU) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    return v;
}
// EPI: the kernel instantiation that applies the output stage (else only
// the store; out_dt is read from e in both)
template <bool EPI>
__device__ __forceinline__ void store_out(void* y, size_t i, size_t n, const Epilogue& e, float v) {
    if constexpr (EPI) v = apply_epilogue(e, n, v);
    store_f(y, i, e.out_dt, v);
}

// code i (0..63) of a 64-code unit held in 2*BITS words w[] (compile-time i
// after unrolling: one v_bfe_u32, or v_alignbit_b32 + and for a straddle)
template <int BITS>
__device__ __forceinline__ uint32_t unit_code(const uint32_t* w, int i) {
    const int bit = i * BITS, wi = bit >> 5, sh = bit & 31;
    const uint32_t mask = (1u << BITS) - 1u;
    if (sh + BITS <= 32) return (w[wi] >> sh) & mask;
    // straddling code: funnel shift (a 64-bit shift can push the word array
    // into a private-memory copy)
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & mask;
}

// Exact 16-bit operand pairs for the dot2 instructions.
//
// For f16 (10 mantissa bits) and bf16 (7 mantissa bits) a code q of BITS
// bits placed in the top BITS mantissa bits of 1.0 gives v(q) = 1 + q*2^-BITS
// exactly.  Then sum_k x_k v(q_k) = xs + 2^-BITS sum_k x_k q_k, and every
// product x_k v(q_k) is exact in fp32 (<= 11 + 9 significant bits).
//
// Where codes sit 16 bits apart inside one word (BITS 2, 4, 8) one shift and
// one v_and_or_b32 build a pair (q_j, q_{j+P/2}) with P = 32/BITS codes per
// word: "apart" pairing, and x is staged in the matching order.  For the
// irregular widths (3, 5, 6) codes are extracted one by one and paired in
// natural order (q_{2p}, q_{2p+1}).
template <int BITS>
struct PairLayout {
    static constexpr bool kApart = (BITS == 2 || BITS == 4 || BITS == 8);
    static constexpr int kCodesPerWord = 32 / BITS;  // meaningful when kApart
};

// position of code k (within its unit-aligned block) in the staged x order
template <int BITS>
__device__ __host__ __forceinline__ int x_slot(int k) {
    if constexpr (PairLayout<BITS>::kApart) {
        constexpr int P = PairLayout<BITS>::kCodesPerWord, H = P / 2;
        int base = k - (k % P), j = k % P;
        return base + (j < H ? 2 * j : 2 * (j - H) + 1);
    } else {
        return k;
    }
}

// gfx9 VOP3 encodings take no literal constants and read at most one SGPR,
// so the compiler splits (x & mask) | magic into v_and + v_or.  These emit
// the fused forms with the mask in an SGPR and the magic in a VGPR.
__device__ __forceinline__ uint32_t vconst(uint32_t c) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(c));
    return v;
}
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t vmagic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(vmagic));
    return r;
}
template <int S>
__device__ __forceinline__ uint32_t lshl_or(uint32_t x, uint32_t vmagic) {
    uint32_t r;
    asm("v_lshl_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "i"(S), "v"(vmagic));
    return r;
}

// Where the operand builder places a code inside each 16-bit half, and the
// factor that maps sum x v(q) back to sum x q.  For BITS 2/4/8 the code LSB
// goes to P, the highest multiple of BITS that leaves the code inside the
// mantissa: one code per word then needs no shift, and v(q) = 1 + q 2^(P-MANT).
// Irregular widths place the code at the top of the mantissa.
template <int BITS, int MANT>
struct MagicCfg {
    static constexpr bool kApart = PairLayout<BITS>::kApart;
    static constexpr int P = kApart ? ((MANT - BITS) / BITS) * BITS : MANT - BITS;
    static constexpr float kPow = (float)(1u << (MANT - P));  // v(q) = 1 + q / kPow
};

// Build the operand pairs of NW words of codes (default: one 64-code unit,
// 32 pairs).  MANT = 10 (f16) or 7 (bf16).
template <int BITS, int MANT, int NW = 2 * BITS>
__device__ __forceinline__ void unit_pairs_magic(const uint32_t* w, uint32_t* pr) {
    using C = MagicCfg<BITS, MANT>;
    constexpr uint32_t one = (MANT == 10) ? 0x3C00u : 0x3F80u;
    const uint32_t magic = vconst(one | (one << 16));
    if constexpr (C::kApart) {
        constexpr int H = PairLayout<BITS>::kCodesPerWord / 2;
        constexpr uint32_t m16 = ((1u << BITS) - 1u) << C::P;
        constexpr uint32_t mask = m16 | (m16 << 16);
#pragma unroll
        for (int wi = 0; wi < NW; wi++) {
#pragma unroll
            for (int j = 0; j < H; j++) {
                // code j of the low half sits at bit j*BITS; move it to P
                const int s = C::P - j * BITS;
                uint32_t r;
                if (s == 0) {
                    r = and_or(w[wi], mask, magic);
                } else if (s > 0) {
                    // mask first, then shift into place and OR the magic
                    r = (w[wi] & (mask >> s));
                    r = (s == 1) ? lshl_or<1>(r, magic) : (s == 2) ? lshl_or<2>(r, magic)
                      : (s == 4) ? lshl_or<4>(r, magic) : (s == 6) ? lshl_or<6>(r, magic)
                      : lshl_or<8>(r, magic);
                } else {
                    r = and_or(w[wi] >> (-s), mask, magic);
                }
                pr[wi * H + j] = r;
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < NW * 16 / BITS; p++) {
            uint32_t lo = unit_code<BITS>(w, 2 * p), hi = unit_code<BITS>(w, 2 * p + 1);
            pr[p] = lshl_or<MANT - BITS>(lo | (hi << 16), magic);
        }
    }
}

// 8-bit codes as bf16 operands: q itself (exact, <= 8 significant bits),
// natural pairing (q_{2p}, q_{2p+1}); NW words (default one 64-code unit).
template <int NW = 16>
__device__ __forceinline__ void unit_pairs_bf16_u8(const uint32_t* w, uint32_t* pr) {
#pragma unroll
    for (int wi = 0; wi < NW; wi++) {
        float f0 = (float)(w[wi] & 0xffu), f1 = (float)((w[wi] >> 8) & 0xffu);
        float f2 = (float)((w[wi] >> 16) & 0xffu), f3 = (float)(w[wi] >> 24);
        // the fp32 values are exact bf16 numbers: keep their upper halves
        pr[2 * wi] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
        pr[2 * wi + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
    }
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c, int tx) {
    if (tx == DT_F16)
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                      false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
}

// ---- wavefront reductions (DPP within 16-lane rows, readlane across rows) --

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// after this every lane of each 16-lane row holds the row's sum
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// full 64-lane sum, wave-uniform result
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

}  // namespace lxq
