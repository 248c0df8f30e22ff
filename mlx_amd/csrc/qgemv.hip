// qgemv.hip -- GEMV dispatch: M chunking and bit-width selection.
#include "qgemv_impl.h"

namespace lxq {
using namespace gemv;

static LuxStatus launch_bits(const QmmArgs& a, hipStream_t st) {
    switch (a.bits) {
    case 2: return launch_b<2>(a, st);
    case 3: return launch_b<3>(a, st);
    case 4: return launch_b<4>(a, st);
    case 5: return launch_b<5>(a, st);
    case 6: return launch_b<6>(a, st);
    case 8: return launch_b<8>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

static LuxStatus launch_mx_bits(const QmmArgs& a, hipStream_t st) {
    switch (a.bits) {
    case 2: return launch_mx_b<2>(a, st);
    case 4: return launch_mx_b<4>(a, st);
    case 8: return launch_mx_b<8>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

// Rows of x that no kernel takes whole are split over launches: four rows
// of 16-bit x per launch of the stream kernel (K <= 4096), two per launch of
// the split-K kernel (K > 4096), one row of f32 x per launch of the M = 1
// kernels.  NotSupported: the generic kernel.
LuxStatus launch_qgemv(const QmmArgs& args, hipStream_t st) {
    if (args.K % 64 != 0) return LuxStatus::NotSupported;
    // rows m0 .. m0 + mc - 1 of x and y
    auto rows = [&](int m0, int mc) {
        QmmArgs a = args;
        a.M = mc;
        const size_t xel = args.x_dtype == DT_F32 ? 4 : 2, yel = args.out_dtype == DT_F32 ? 4 : 2;
        a.x = static_cast<const uint8_t*>(args.x) + (size_t)m0 * args.K * xel;
        a.y = static_cast<uint8_t*>(args.y) + (size_t)m0 * args.N * yel;
        return a;
    };
    // 2..16 rows of x: the MFMA kernels where they apply (16-bit x; the
    // decode kernel takes 4-bit codes and M <= 8, the LDS-ring kernel 4/8-bit
    // codes; both need K % 1024 == 0), except where the stream kernel (M <= 4,
    // K <= 4096) or the skinny one measured faster (graph replays):
    //  - M = 2, 16-bit x, K <= 4096: 4-bit 11.1 us against 11.5 at K = 4096,
    //    N = 14336; 8.0 against 11.0 at N = 11008; 4.9 against 5.9 at N = 4096;
    //  - 8-bit codes, M <= 8, K <= 4096 (LDS-ring kernel skipped): M = 3 / 4 /
    //    6 / 8 at K = 4096, N = 14336: 18.1 / 19.5 / 19.9 / 20.1 us against
    //    22.7 / 22.9 / 23.1 / 23.2; M = 4, N = 4096: 7.2 against 10.5 (at
    //    K = 8192 the LDS-ring kernel stays: 20.2 against 25.0).
    //  - M = 2, 16-bit x, 8192 < K <= 16384: the split-K stream kernel
    //    (K = 14336, N = 4096: 18.1 us against 25.7 on the LDS-ring kernel;
    //    8-bit K = 12288: 17.7 against 25.3); at K <= 8192 the decode kernel
    //    is faster (K = 8192, N = 8192: 12.8 against 18.1).
    // 2..4 rows of x with K <= 16384: the K-split whole-line kernel where it
    // applies and measured faster (qgemv_mx.h, mx_wins: f32 x; every K > 8192;
    // M = 2 and 2-bit codes up to K = 8192; at K <= 4096 8-bit codes, 2-bit at
    // M >= 3, 4-bit at M = 2 with f16 x)
    // 4-bit codes: the 4x4x4-MFMA decode kernel (K = 2048, 4096, 8192) at
    // M <= 4, and at M = 5..8 with K = 4096 (two x sets; at K = 2048 and
    // 8192 the decode kernel stays faster there).  Same box, us per launch
    // against the kernels AUTO picked before: K = 4096, N = 14336, M = 2 / 3
    // / 4 / 6 / 8 8.8 / 9.1 / 9.0 / 11.7 / 12.1 against 10.2 / 12.1 / 12.2 /
    // 12.6 / 13.0; K = N = 8192 M = 4 12.2 against 13.8 (M = 8 20.1 against
    // 15.0); K = 2048, N = 8192, M = 8 5.6 against 5.4.  At M <= 4 it also
    // takes 8192 < K <= 16384 (two chunks per lane) from the K-split
    // whole-line kernel: K = 14336, N = 4096, M = 2 / 3 / 4 9.9 / 10.5 / 11.2
    // against 11.9 / 16.1 / 16.2; K = 11008 8.6 / 9.0 / 9.5 against 11.2 /
    // 15.6 / 15.6 (qgemv_q4.hip)
    if (args.M >= 2 && args.bits == 4 && (args.M <= 4 || (args.M <= 8 && args.K == 4096))) {
        const LuxStatus s = launch_qgemv_q4(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    // 5..8 rows of x, 16-bit x, 8192 < K <= 16384: rows 0..3 and the rest as
    // two launches of the kernels above (the second finds W in the Infinity
    // Cache) where the LDS-ring kernel does not take the shape (K % 1024 !=
    // 0, 2-bit codes) or fills half the CUs (4-bit, N <= 4096; its 32-row
    // blocks).  Same box, g64, N = 4096, M = 5 / 6 / 8, us per launch: K =
    // 11008, 4-bit 32.3 / 35.5 / 46.8 -> 18.5 / 17.5 / 18.7 (split-K kernel
    // before), 8-bit 37.8 / 41.1 / 54.1 -> 32.1 / 34.7 / 39.3; K = 14336,
    // 2-bit 34.4 / 41.0 / 54.4 -> 23.1 / 25.0 / 29.5, 4-bit 25.4 / 25.5 /
    // 25.4 -> 21.2 / 21.5 / 23.0 (LDS-ring kernel before).  Not taken: 8-bit
    // at K = 14336 (27.4 -> 33.9..40.7) and 4-bit at N = 8192 (27.5 ->
    // 37.8..44.9), where the LDS-ring kernel fills the CUs.
    if (args.M >= 5 && args.M <= 8 && args.x_dtype != DT_F32 && args.K > 8192 && args.K <= 16384 &&
        (args.bits == 2 || args.bits == 4 || args.bits == 8) &&
        (args.K % 1024 != 0 || args.bits == 2 || (args.bits == 4 && args.N <= 4096))) {
        const LuxStatus s = launch_qgemv(rows(0, 4), st);
        if (s != LuxStatus::Ok) return s;
        return launch_qgemv(rows(4, args.M - 4), st);
    }
    if (args.M >= 2 && args.M <= 4) {
        const LuxStatus s = launch_mx_bits(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    const bool stream2 = args.M == 2 && args.x_dtype != DT_F32 && (args.K <= 4096 || (args.K > 8192 && args.K <= 16384));
    const bool ring8 = !(args.bits == 8 && args.M <= 8 && args.K <= 4096);
    if (args.M >= 2 && args.M <= 8 && !stream2) {
        const LuxStatus s = launch_qgemv_dec(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    if (args.M >= 2 && args.M <= 16 && !stream2 && ring8) {
        const LuxStatus s = launch_qgemv_mid(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    if (args.M >= 5 && args.M <= 16) {
        const LuxStatus s = launch_qmm_skinny(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    // f32 x, two rows or more, where the K-split whole-line kernel does not
    // run (3/5/6-bit codes; K > 16384; K not a whole number of its waves'
    // 16-code steps, launch_mx_b): one launch of the M = 1 kernels per
    // row (whole-line or stream up to K = 4096, split-K up to 32768) instead
    // of the row-run kernel (since retired), or the generic kernel where one
    // row of f32 x overflowed that kernel's staging (K >= 18944).  Same box, g64,
    // f32 x, scales and output, us per launch, K = 4096, N = 14336, M = 2 /
    // 3 / 4 / 8: 3-bit 35.6 / 45.6 / 68.3 / 133.4 -> 17.6 / 26.0 / 34.5 /
    // 68.0; 5-bit 56.5 / 72.0 / 114.9 / 224.2 -> 22.1 / 32.8 / 43.3 / 86.0;
    // 6-bit 57.0 / 70.2 / 116.4 / 227.5 -> 23.4 / 34.4 / 45.8 / 88.8 (N =
    // 4096: 40-52 % less).  Every row is the same launch, so the gain holds
    // at any M.
    if (args.x_dtype == DT_F32 && args.M >= 2 &&
        (args.bits == 3 || args.bits == 5 || args.bits == 6 || args.K > 16384 ||
         args.K % (16 * (args.K > 8192 ? 16 : args.K > 4096 ? 8 : 4)) != 0)) {
        for (int m0 = 0; m0 < args.M; m0++) {
            const LuxStatus s = launch_bits(rows(m0, 1), st);
            if (m0 == 0 && s == LuxStatus::NotSupported) break;  // nothing launched: the kernels below
            if (s != LuxStatus::Ok) return s;
            if (m0 + 1 == args.M) return LuxStatus::Ok;
        }
    }
    // one or two rows of x: the whole-line, stream and split-K kernels take
    // them whole (the split-K kernel stages both x rows itself, up to
    // K = 16384); only if they decline, the row chunks below
    if (args.M <= 2) {
        const LuxStatus s = launch_bits(args, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    // f32 x with more than 4 rows: chunks of 4 (a last single row on the
    // M = 1 kernels) on the K-split whole-line kernel where it applies
    // (M = 8, K = 4096, N = 14336, 4-bit: the row-run kernel took 126.9 us)
    if (args.x_dtype == DT_F32 && args.M > 4) {
        for (int m0 = 0; m0 < args.M; m0 += 4) {
            const QmmArgs a = rows(m0, args.M - m0 < 4 ? args.M - m0 : 4);
            const LuxStatus s = a.M >= 2 ? launch_mx_bits(a, st) : launch_bits(a, st);
            if (m0 == 0 && s == LuxStatus::NotSupported) break;  // nothing launched: the row chunks below
            if (s != LuxStatus::Ok) return s;
            if (m0 + 4 >= args.M) return LuxStatus::Ok;
        }
    }
    // 16-bit x, K > 4096, three rows or more that no kernel above took:
    // pairs of rows on the split-K kernel (a last single row on the M = 1
    // kernels) rather than a row-run kernel (since retired) in chunks of up to 4 rows, or
    // the generic kernel where one row of x overflows its 64 KB staging.
    // Same box, g64, us per launch: K = 5120, N = 13824, 3-bit, M = 3 / 4 /
    // 8: 81.8 / 99.5 / 186.7 -> 36.3 / 41.8 / 82.6 (5/6-bit alike); K =
    // 6144, N = 4096, M = 4: 36.0 -> 16.3; 4-bit K = 6656 40.6 -> 15.8; K =
    // 28672, N = 8192, 3-bit M = 3 / 8: 17132 / 24198 -> 92.7 / 238.5
    if (args.x_dtype != DT_F32 && args.K > 4096 && args.M > 2) {
        for (int m0 = 0; m0 < args.M; m0 += 2) {
            const LuxStatus s = launch_bits(rows(m0, args.M - m0 < 2 ? 1 : 2), st);
            if (m0 == 0 && s == LuxStatus::NotSupported) break;  // nothing launched: the chunks below
            if (s != LuxStatus::Ok) return s;
            if (m0 + 2 >= args.M) return LuxStatus::Ok;
        }
    }
    // the rest (16-bit x at K <= 4096: 3/5/6-bit codes and the shapes the
    // kernels above decline): chunks of 4 rows on the stream kernel, the last
    // one 1..4 rows.  They ran in one launch of a row-run kernel with up to 8
    // rows of x staged in LDS, since retired (same box, g64, us per launch,
    // M = 8, K = 2048, N = 8192: 3-bit 55.9 -> 16.2, 2-bit 56.0 -> 15.4; M =
    // 6, K = 3072, N = 14336, 5-bit 83.9 -> 26.0; 8-bit N = 8192 60.7 ->
    // 14.9).  Anything else is NotSupported here: the generic kernel.
    for (int m0 = 0; m0 < args.M; m0 += 4) {
        const LuxStatus s = launch_bits(rows(m0, args.M - m0 < 4 ? args.M - m0 : 4), st);
        if (s != LuxStatus::Ok) return s;
    }
    return LuxStatus::Ok;
}

}  // namespace lxq
