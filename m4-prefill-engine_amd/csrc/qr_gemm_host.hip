// qr_gemm_host.hip -- host side of the tiled projection: format dispatch,
// split-K choice and workspace sizing (kernels in qr_gemm.hip), and the
// split-K reduction kernel shared with the small-M kernel.
#include "qr_device.h"
#include "qr_gemm_shapes.h"

namespace qr {

// Split-K reduction: out[m, n] = epilogue(sum over splits z = 0, 1, ... of
// ws[z][plane][m][n]) with the tiled kernel's epilogue arithmetic (SwiGLU
// silu(g) u in fp32 for DUAL, + fp16 residual, one rounding to fp16,
// [M, N] or head-major [N / head_D, M, head_D]).  The splits are summed in
// split order starting from 0, so the result does not depend on which
// workgroup finished first.  Eight consecutive elements of one row per
// thread (16-byte output stores) when N and head_D are multiples of 8 and Y
// and R are 16-byte aligned; the
// partials are read once, as streaming loads.
constexpr int kRedVec = 8;

template <bool DUAL>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ ws, uint32_t ks, uint32_t M,
                                                            uint32_t N, const _Float16* __restrict__ R,
                                                            _Float16* __restrict__ Y, uint32_t head_D) {
    const size_t plane = (size_t)M * N;
    const size_t e0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * kRedVec;
    if (e0 >= plane) return;
    const int cnt = plane - e0 < (size_t)kRedVec ? (int)(plane - e0) : kRedVec;
    const bool vec = cnt == kRedVec && (N % kRedVec) == 0 && (head_D % kRedVec) == 0 &&
                     ((reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(R)) & 15u) == 0;
    float g[kRedVec], u[kRedVec];
#pragma unroll
    for (int q = 0; q < kRedVec; q++) g[q] = u[q] = 0.0f;
    if (vec) {
        for (uint32_t z = 0; z < ks; z++) {
            const f4_t* src = reinterpret_cast<const f4_t*>(ws + (size_t)z * plane * (DUAL ? 2 : 1) + e0);
            const f4_t a0 = __builtin_nontemporal_load(src), a1 = __builtin_nontemporal_load(src + 1);
            g[0] += a0.x; g[1] += a0.y; g[2] += a0.z; g[3] += a0.w;
            g[4] += a1.x; g[5] += a1.y; g[6] += a1.z; g[7] += a1.w;
            if constexpr (DUAL) {
                const f4_t* sv = reinterpret_cast<const f4_t*>(reinterpret_cast<const float*>(src) + plane);
                const f4_t b0 = __builtin_nontemporal_load(sv), b1 = __builtin_nontemporal_load(sv + 1);
                u[0] += b0.x; u[1] += b0.y; u[2] += b0.z; u[3] += b0.w;
                u[4] += b1.x; u[5] += b1.y; u[6] += b1.z; u[7] += b1.w;
            }
        }
        const uint32_t m = (uint32_t)(e0 / N), n = (uint32_t)(e0 % N);
        float v[kRedVec];
#pragma unroll
        for (int q = 0; q < kRedVec; q++) {
            v[q] = g[q];
            if constexpr (DUAL) v[q] = silu_mul(v[q], u[q]);
        }
        if (R) {
            const u4_t rr = *reinterpret_cast<const u4_t*>(R + e0);
            const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const h2_t hh = as_h2(rw[q]);
                v[2 * q] += (float)hh.x;
                v[2 * q + 1] += (float)hh.y;
            }
        }
        const size_t o = head_D ? ((size_t)(n / head_D) * M + m) * head_D + n % head_D : e0;
        u4_t out;
        out.x = pack_h2(f2h_bits(v[0]), f2h_bits(v[1]));
        out.y = pack_h2(f2h_bits(v[2]), f2h_bits(v[3]));
        out.z = pack_h2(f2h_bits(v[4]), f2h_bits(v[5]));
        out.w = pack_h2(f2h_bits(v[6]), f2h_bits(v[7]));
        *reinterpret_cast<u4_t*>(Y + o) = out;
        return;
    }
    for (uint32_t z = 0; z < ks; z++) {
        const float* src = ws + (size_t)z * plane * (DUAL ? 2 : 1) + e0;
        for (int q = 0; q < cnt; q++) {
            g[q] += src[q];
            if constexpr (DUAL) u[q] += src[plane + q];
        }
    }
    for (int q = 0; q < cnt; q++) {
        const size_t e = e0 + q;
        const uint32_t m = (uint32_t)(e / N), n = (uint32_t)(e % N);
        float v = g[q];
        if constexpr (DUAL) v = silu_mul(v, u[q]);
        if (R) v += (float)R[e];
        const size_t o = head_D ? ((size_t)(n / head_D) * M + m) * head_D + n % head_D : e;
        Y[o] = (_Float16)v;
    }
}

hipError_t launch_splitk_reduce(const float* ws, uint32_t ks, uint32_t M, uint32_t N, bool dual, const _Float16* R,
                                _Float16* Y, uint32_t head_D, hipStream_t st) {
    const size_t plane = (size_t)M * N;
    const unsigned blocks = (unsigned)((plane + 256 * kRedVec - 1) / (256 * kRedVec));
    if (dual)
        hipLaunchKernelGGL(splitk_reduce_kernel<true>, dim3(blocks), dim3(256), 0, st, ws, ks, M, N, R, Y, head_D);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<false>, dim3(blocks), dim3(256), 0, st, ws, ks, M, N, R, Y, head_D);
    return hipGetLastError();
}

static hipError_t launch_gemm_main(const GemmParams& p, hipStream_t st) {
    switch (p.format) {
        case QUANT_Q4_0: return launch_gemm_format<QUANT_Q4_0>(p, st);
        case QUANT_MLX_4BIT: return launch_gemm_format<QUANT_MLX_4BIT>(p, st);
        case QUANT_Q4_K: return launch_gemm_format<QUANT_Q4_K>(p, st);
        case QUANT_TERNARY_1_58: return launch_gemm_format<QUANT_TERNARY_1_58>(p, st);
        case QUANT_VAR_RATE_AFFINE: return launch_gemm_format<QUANT_VAR_RATE_AFFINE>(p, st);
        case QUANT_EXL3: return launch_gemm_format<QUANT_EXL3>(p, st);
        case QUANT_Q8_0: return launch_gemm_format<QUANT_Q8_0>(p, st);
        case QUANT_PRISM_Q2_0: return launch_gemm_format<QUANT_PRISM_Q2_0>(p, st);
        case QUANT_MLX_4BIT_G64: return launch_gemm_format<QUANT_MLX_4BIT_G64>(p, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const GemmParams& p0, hipStream_t st) {
    GemmParams p = p0;
    p.group_m = gemm_group_m(p);
    hipError_t e = launch_gemm_main(p, st);
    if (e == hipSuccess && p.ksplit > 1)
        e = launch_splitk_reduce(p.ws, p.ksplit, p.M, p.N, p.W2 != nullptr, p.R, p.Y, p.head_D, st);
    return e;
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
    const int s0 = rb_pick(p.format, p.M, p.N, p.K, false);
    for (uint32_t g = 1; g < p.ngroups; g++)
        if (rb_pick(p.format, p.M, p.Nx[g - 1], p.K, false) != s0) return false;
    return gemm_pick_ksplit(p) == 1;
}

uint32_t gemm_pick_ksplit(const GemmParams& p) {
    const int shape = rb_pick(p.format, p.M, p.N, p.K, p.W2 != nullptr);
    if (shape == 5 || shape == 6) return 1;  // K groups: the tile takes the whole K range
    const RbShape d = rb_dims(shape);
    const uint32_t T = tiles_of(p, d);
    // One workgroup fits a CU (its registers), so the grid runs in waves of
    // 256 workgroups: split K (powers of two, whole 256-element super-blocks,
    // >= 512 of K per split) while the grid still fits one such wave.
    uint32_t ks = 1;
    while (T * ks * 2 <= 256 && p.K % (256 * ks * 2) == 0 && p.K / (ks * 2) >= 512) ks *= 2;
    return ks;
}

size_t gemm_workspace_floats(const GemmParams& p, uint32_t ks) {
    return ks > 1 ? (size_t)ks * p.M * p.N * (p.W2 != nullptr ? 2 : 1) : 0;
}

uint32_t gemm_group_m(const GemmParams& p) {
    const RbShape d = rb_dims(rb_pick(p.format, p.M, p.N, p.K, p.W2 != nullptr));
    const uint32_t nt_m = (p.M + d.bm - 1) / d.bm;
    return nt_m >= 4 ? 4u : 2u;
}

}  // namespace qr
