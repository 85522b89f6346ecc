// qr_gemm_host.hip -- host side of the tiled projection: format dispatch,
// split-K choice and workspace sizing (kernels in qr_gemm.hip).
#include "qr_gemm_shapes.h"

namespace qr {

hipError_t launch_gemm(const GemmParams& p0, hipStream_t st) {
    GemmParams p = p0;
    p.group_m = gemm_group_m(p);
    switch (p.format) {
        case QUANT_Q4_0: return launch_gemm_format<QUANT_Q4_0>(p, st);
        case QUANT_MLX_4BIT: return launch_gemm_format<QUANT_MLX_4BIT>(p, st);
        case QUANT_Q4_K: return launch_gemm_format<QUANT_Q4_K>(p, st);
        case QUANT_TERNARY_1_58: return launch_gemm_format<QUANT_TERNARY_1_58>(p, st);
        case QUANT_VAR_RATE_AFFINE: return launch_gemm_format<QUANT_VAR_RATE_AFFINE>(p, st);
        case QUANT_EXL3: return launch_gemm_format<QUANT_EXL3>(p, st);
        case QUANT_Q8_0: return launch_gemm_format<QUANT_Q8_0>(p, st);
        case QUANT_PRISM_Q2_0: return launch_gemm_format<QUANT_PRISM_Q2_0>(p, st);
        default: return hipErrorInvalidValue;
    }
}

static uint32_t tiles_of(const GemmParams& p, const RbShape& d) {
    const uint32_t ntm = (p.M + d.bm - 1) / d.bm;
    uint32_t T = ntm * ((p.N + d.bn - 1) / d.bn);
    for (uint32_t g = 1; g < p.ngroups && g < 3; g++) T += ntm * ((p.Nx[g - 1] + d.bn - 1) / d.bn);
    return T;
}

bool gemm_grouped_ok(const GemmParams& p) {
    if (p.ngroups < 2 || p.ngroups > 3 || p.W2 || p.R) return false;
    // every group must take the shape group 0 takes, and the grid needs no K split
    const int s0 = rb_pick(p.format, p.M, p.N, false);
    for (uint32_t g = 1; g < p.ngroups; g++)
        if (rb_pick(p.format, p.M, p.Nx[g - 1], false) != s0) return false;
    return gemm_pick_ksplit(p) == 1;
}

uint32_t gemm_pick_ksplit(const GemmParams& p) {
    const RbShape d = rb_dims(rb_pick(p.format, p.M, p.N, p.W2 != nullptr));
    const uint32_t T = tiles_of(p, d);
    // One workgroup fits a CU (its registers), so the grid runs in waves of
    // 256 workgroups: split K (powers of two, whole 256-element super-blocks,
    // >= 512 of K per split) while the grid still fits one such wave.
    uint32_t ks = 1;
    while (T * ks * 2 <= 256 && p.K % (256 * ks * 2) == 0 && p.K / (ks * 2) >= 512) ks *= 2;
    return ks;
}

size_t gemm_workspace_floats(const GemmParams& p, uint32_t ks, uint32_t* tiles) {
    const bool dual = p.W2 != nullptr;
    const RbShape d = rb_dims(rb_pick(p.format, p.M, p.N, dual));
    const uint32_t T = ((p.M + d.bm - 1) / d.bm) * ((p.N + d.bn - 1) / d.bn);
    if (tiles) *tiles = T;
    return ks > 1 ? (size_t)ks * T * d.bm * d.bn * (dual ? 2 : 1) : 0;
}

uint32_t gemm_group_m(const GemmParams& p) {
    const RbShape d = rb_dims(rb_pick(p.format, p.M, p.N, p.W2 != nullptr));
    const uint32_t nt_m = (p.M + d.bm - 1) / d.bm;
    return nt_m >= 4 ? 4u : 2u;
}

}  // namespace qr
