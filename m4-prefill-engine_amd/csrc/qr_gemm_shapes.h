// qr_gemm_shapes.h -- tile shapes of the tiled projection kernel (qr_gemm.hip),
// shared by the per-format kernel units and the host-side launch helpers.
#pragma once
#include "qr_formats.h"
#include "qr_kernels.h"

namespace qr {

// Shapes {TM, TN, NW, WR, KG}: NW waves in KG K groups of WR row groups;
// BM = 32 TM WR, BN = 32 TN NW / (WR KG).
//   0 (M >= 1024): QR_RB_BIG  (4, 2, 4 -> 128 x 256; Q4_K and ternary:
//                  QR_RB_BIG_K, 4, 1, 8 -> 128 x 256 with two waves per
//                  SIMD, whose heavier decode then overlaps the other wave's MFMAs)
//   1 (M <  1024): QR_RB_MID  (4, 1, 4 -> 128 x 128: twice the tiles
//                  of 128 x 256 at the same K split, half the reduction)
//   4 (M <  1024, last 128-row tile at most half full, cheap-decode formats):
//                  QR_RB_MID64 (2, 1, 4 -> 64 x 128: e.g. M = 129
//                  computes 192 rows, not 256)
//   6 (as 4, no K split needed): QR_RB_MID64_KG (2, 1, 8, 1, 2 -> 64 x 128 as
//                  two K groups of four column waves)
//   5 (M <= 128, wide N): QR_RB_KG (4, 1, 4, 1, 2 -> 128 x 64: two K groups
//                  of two column waves take alternate K steps and meet in LDS,
//                  so 224 workgroups cover M = 128, N = 14336 with no K split)
//   dual (SwiGLU): 4, 1, 4 -> 128 x 128 outputs (gate + up: 256 weight columns)
#define QR_RB_BIG 4, 2, 4, 1, 1
#define QR_RB_BIG_K 4, 1, 8, 1, 1
#define QR_RB_MID 4, 1, 4, 1, 1
#define QR_RB_MID64 2, 1, 4, 1, 1
#define QR_RB_KG 4, 1, 4, 1, 2
#define QR_RB_MID64_KG 2, 1, 8, 1, 2
#define QR_RB_DUAL 4, 1, 4, 1, 1
template <int TM, int TN, int NW, int WR, int KG> struct ShapeOf {
    static constexpr uint32_t bm = 32 * TM * WR, bn = 32 * TN * (NW / (WR * KG));
};
struct RbShape {
    uint32_t bm, bn;
};
// Shape choice.  At M >= 1024 the wide tile is used while it alone fills the
// 256 CUs; when it cannot (N small), 128 x 128 tiles give twice the tiles, so
// the K split -- whose fp32 partials are M x N x 4 bytes written and read per
// extra split -- is halved or avoided.
inline int rb_pick(int format, uint32_t M, uint32_t N, uint32_t K, bool dual) {
    if (dual) return 2;
    // The 3/5-bit double-rounding formats (no BASELINE configuration) keep
    // one tile shape: fewer instances of their heavy fp64 decode to compile.
    if (format == QUANT_VAR_RATE_AFFINE || format == QUANT_EXL3) return 1;
    // K groups instead of a K split: one 128-row tile, enough 64-column tiles
    // for most of the CUs, whole pairs of 64-K steps
    if (M <= 128 && (N + 63) / 64 >= 192 && K % 128 == 0) return 5;
    if (M >= 1024) {
        // the heavier decodes (Q4_K's fp32 affine, ternary's 2-bit fields) run
        // best as two waves per SIMD, one decoding while the other multiplies
        // (ternary M = 2048: 68-70 us vs 76 us with one wave per SIMD)
        if (format == QUANT_Q4_K || format == QUANT_TERNARY_1_58) return 3;
        const uint32_t big_tiles = ((M + 127) / 128) * ((N + 255) / 256);
        if (big_tiles < 256) return 1;
        return 0;
    }
    // 64-row tiles decode every weight twice as often per MFMA: worth it only
    // for the formats with a cheap decode (measured at M = 129: Q4_0, MLX and
    // ternary 6-20% faster, Q4_K 8-9% slower)
    const bool cheap = format == QUANT_Q4_0 || format == QUANT_MLX_4BIT || format == QUANT_TERNARY_1_58 ||
                       format == QUANT_Q8_0 || format == QUANT_PRISM_Q2_0 || format == QUANT_MLX_4BIT_G64;
    const uint32_t tail = M % 128;
    if (cheap && tail != 0 && tail <= 64) {
        // the same tile as two K groups of four waves (two per SIMD, each
        // taking alternate steps: half the serial steps per wave) when the
        // grid needs no K split anyway (cfg4: 15.6 -> 14.5 us)
        if (K % 128 == 0 && ((M + 63) / 64) * ((N + 127) / 128) > 128) return 6;
        return 4;
    }
    return 1;
}
inline RbShape rb_dims(int s) {
    switch (s) {
        case 0: return {ShapeOf<QR_RB_BIG>::bm, ShapeOf<QR_RB_BIG>::bn};
        case 3: return {ShapeOf<QR_RB_BIG_K>::bm, ShapeOf<QR_RB_BIG_K>::bn};
        case 1: return {ShapeOf<QR_RB_MID>::bm, ShapeOf<QR_RB_MID>::bn};
        case 4: return {ShapeOf<QR_RB_MID64>::bm, ShapeOf<QR_RB_MID64>::bn};
        case 5: return {ShapeOf<QR_RB_KG>::bm, ShapeOf<QR_RB_KG>::bn};
        case 6: return {ShapeOf<QR_RB_MID64_KG>::bm, ShapeOf<QR_RB_MID64_KG>::bn};
        default: return {ShapeOf<QR_RB_DUAL>::bm, ShapeOf<QR_RB_DUAL>::bn};
    }
}

// Launches the tiled kernel of format F (plain, or the SwiGLU dual variant when
// p.W2 is set); one explicit instantiation per format, each in its own
// compilation unit (qr_gemm.hip built with -DQR_GEMM_FORMAT=F).
template <int F>
hipError_t launch_gemm_format(const GemmParams& p, hipStream_t st);

}  // namespace qr
