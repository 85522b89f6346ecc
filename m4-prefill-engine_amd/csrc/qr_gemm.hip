// qr_gemm.hip -- quantized projection Y = X . W^T on gfx950 MFMA.
//
// Replaces the reference's block_mma_64x64_engine (quant_router_kernels.metal:
// 442-581) and its 14 entry points (:588-927), and the fused dual-projection
// SwiGLU swiglu_mma_dual_simd (brick3_swiglu_kernels.metal:428-698).
//
// Design (one workgroup = 4 wave64s, one BM x BN output tile):
//  * K advances 64 per step (two 32-element weight groups per column).
//  * X tile [BM x 64] fp16 is loaded with 16-byte buffer loads; the weight
//    groups of the BN columns are loaded raw (compressed) and decoded in
//    registers to binary16 (qr_decode.h, bit-exact vs the CPU unpack), then
//    both are written to a double-buffered LDS stage.  Loads for step k+1 are
//    issued before the MFMAs of step k, so the HBM latency hides under MFMA.
//  * Each wave computes a (TM*32) x (TN*32) sub-tile with
//    v_mfma_f32_32x32x16_f16 (fp32 accumulation).  Both operands are
//    K-contiguous in LDS, so every lane fetches its 8 halfs with one
//    ds_read_b128; rows are padded by 8 halfs to spread LDS banks.
//  * Epilogue: fp32 accumulator (+ optional fp16 residual, + SwiGLU for the
//    dual variant) rounded once to fp16, written [M, N] or head-major
//    [H, M, D] (direct-head routing, quant_router_kernels.metal:570-574).
#include "qr_decode.h"
#include "qr_kernels.h"

namespace qr {

constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;  // halfs per LDS row (padding vs bank conflicts)

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL>
struct GemmCfg {
    static constexpr int BM = WGM * TM * 32;
    static constexpr int BN = WGN * TN * 32;
    static constexpr int NCOL = DUAL ? 2 * BN : BN;       // weight columns decoded per step
    static constexpr int UNITS = NCOL * 2;                // 32-element groups per step
    static constexpr int UPT = (UNITS + 255) / 256;       // groups per thread
    static constexpr int XCH = BM * kBK / 8;              // 16-byte X chunks per step
    static constexpr int XPT = (XCH + 255) / 256;
    static constexpr int LDS_A = BM * kLdsRow;            // halfs per stage
    static constexpr int LDS_B = NCOL * kLdsRow;
    static constexpr int LDS_STAGE = LDS_A + LDS_B;
    static_assert(WGM * WGN == 4, "4 waves per workgroup");
};

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL>
__global__ void __launch_bounds__(256)
gemm_kernel(GemmParams p) {
    using C = GemmCfg<F, WGM, WGN, TM, TN, DUAL>;
    using Dec = Decoder<F>;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    // Grid: x = N tiles, y = M tiles.
    const int n0 = blockIdx.x * C::BN;
    const int m0 = blockIdx.y * C::BM;
    const uint32_t K = p.K;
    const uint32_t nsteps = (K + kBK - 1) / kBK;
    const uint32_t ngroups = K / 32;                       // 32-element groups per column
    const uint32_t col_bytes = (uint32_t)p.col_bytes;

    // Buffer resources: X rows of this tile; W columns of this tile.
    const int mrows = min(C::BM, (int)p.M - m0);
    const int ncols = min(C::BN, (int)p.N - n0);
    auto xr = make_rsrc(p.X + (size_t)m0 * K, (uint32_t)mrows * K * 2u);
    auto wr0 = make_rsrc(p.W + (size_t)n0 * col_bytes, (uint32_t)ncols * col_bytes);
    auto wr1 = make_rsrc(DUAL ? p.W2 + (size_t)n0 * col_bytes : p.W, DUAL ? (uint32_t)ncols * col_bytes : 0u);

    uint32_t xraw[C::XPT][4];
    uint32_t wraw[C::UPT][Dec::kRawWords];

    auto load_step = [&](uint32_t step) {
        const uint32_t k0 = step * kBK;
#pragma unroll
        for (int i = 0; i < C::XPT; i++) {
            int c = tid + 256 * i;
            int row = c >> 3, kc = c & 7;
            uint32_t k = k0 + kc * 8;
            uint32_t off = (c < C::XCH && k < K) ? ((uint32_t)row * K + k) * 2u : kOOB;
            u4_t v = ld_b128(xr, off);
            xraw[i][0] = v.x; xraw[i][1] = v.y; xraw[i][2] = v.z; xraw[i][3] = v.w;
        }
#pragma unroll
        for (int u = 0; u < C::UPT; u++) {
            int unit = tid + 256 * u;
            int col = unit >> 1;
            uint32_t g = step * 2 + (unit & 1);
            bool dual_up = DUAL && col >= C::BN;
            int lcol = dual_up ? col - C::BN : col;
            uint32_t coff = (unit < C::UNITS && g < ngroups && lcol < ncols) ? (uint32_t)lcol * col_bytes : kOOB;
            if (coff == kOOB) {
#pragma unroll
                for (int j = 0; j < Dec::kRawWords; j++) wraw[u][j] = 0;
            } else {
                Dec::load(dual_up ? wr1 : wr0, coff, g, wraw[u]);
            }
        }
    };

    auto store_step = [&](uint32_t step, int stage) {
        _Float16* As = lds + stage * C::LDS_STAGE;
        _Float16* Bs = As + C::LDS_A;
#pragma unroll
        for (int i = 0; i < C::XPT; i++) {
            int c = tid + 256 * i;
            if (c < C::XCH) {
                int row = c >> 3, kc = c & 7;
                u4_t v = {xraw[i][0], xraw[i][1], xraw[i][2], xraw[i][3]};
                *reinterpret_cast<u4_t*>(As + row * kLdsRow + kc * 8) = v;
            }
        }
#pragma unroll
        for (int u = 0; u < C::UPT; u++) {
            int unit = tid + 256 * u;
            if (unit < C::UNITS) {
                int col = unit >> 1;
                uint32_t g = step * 2 + (unit & 1);
                int lcol = (DUAL && col >= C::BN) ? col - C::BN : col;
                uint32_t out[16];
                if (g < ngroups && lcol < ncols) {
                    Dec::decode(wraw[u], Dec::parity((uint32_t)lcol * col_bytes, g), out);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; j++) out[j] = 0;
                }
                u4_t* dst = reinterpret_cast<u4_t*>(Bs + col * kLdsRow + (unit & 1) * 32);
#pragma unroll
                for (int j = 0; j < 4; j++) dst[j] = u4_t{out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]};
            }
        }
    };

    f16v_t acc[TM][TN];
    f16v_t acc2[DUAL ? TM : 1][DUAL ? TN : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f16v_t{};
    if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc2[i][j] = f16v_t{};
    }

    load_step(0);
    store_step(0, 0);
    __syncthreads();

    const int arow = wm * TM * 32 + (lane & 31);
    const int bcol = wn * TN * 32 + (lane & 31);
    const int kq = (lane >> 5) * 8;

    for (uint32_t s = 0; s < nsteps; s++) {
        const int stage = s & 1;
        if (s + 1 < nsteps) load_step(s + 1);
        const _Float16* As = lds + stage * C::LDS_STAGE;
        const _Float16* Bs = As + C::LDS_A;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; kk++) {
            h8_t a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const h8_t*>(As + (arow + i * 32) * kLdsRow + kk * 16 + kq);
#pragma unroll
            for (int j = 0; j < TN; j++)
                b[j] = *reinterpret_cast<const h8_t*>(Bs + (bcol + j * 32) * kLdsRow + kk * 16 + kq);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            if constexpr (DUAL) {
                h8_t b2[TN];
#pragma unroll
                for (int j = 0; j < TN; j++)
                    b2[j] = *reinterpret_cast<const h8_t*>(Bs + (C::BN + bcol + j * 32) * kLdsRow + kk * 16 + kq);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b2[j], acc2[i][j], 0, 0, 0);
            }
        }
        if (s + 1 < nsteps) store_step(s + 1, stage ^ 1);
        __syncthreads();
    }

    // Epilogue.  Accumulator element r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
    // column l%32 of the 32x32 MFMA tile.
    const uint32_t M = p.M, N = p.N;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * TN * 32 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * TM * 32 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < (int)M && n < (int)N) {
                    float v = acc[i][j][r];
                    if constexpr (DUAL) {
                        float u = acc2[i][j][r];
                        v = v / (1.0f + __expf(-v)) * u;
                    }
                    if (p.R) v += (float)p.R[(size_t)m * N + n];
                    size_t o;
                    if (p.head_D) {
                        uint32_t h = (uint32_t)n / p.head_D, dd = (uint32_t)n % p.head_D;
                        o = ((size_t)h * M + m) * p.head_D + dd;
                    } else {
                        o = (size_t)m * N + n;
                    }
                    p.Y[o] = (_Float16)v;
                }
            }
        }
}

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL>
static hipError_t launch_cfg(const GemmParams& p, hipStream_t st) {
    using C = GemmCfg<F, WGM, WGN, TM, TN, DUAL>;
    auto kern = gemm_kernel<F, WGM, WGN, TM, TN, DUAL>;
    const size_t lds = 2 * C::LDS_STAGE * sizeof(_Float16);
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    dim3 grid((p.N + C::BN - 1) / C::BN, (p.M + C::BM - 1) / C::BM);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, p);
    return hipGetLastError();
}

template <int F, bool DUAL>
static hipError_t launch_fmt(const GemmParams& p, hipStream_t st) {
    if (DUAL) {
        if (p.M <= 32) return launch_cfg<F, 1, 4, 1, 1, DUAL>(p, st);
        return launch_cfg<F, 2, 2, 2, 1, DUAL>(p, st);
    }
    if (p.M <= 32) return launch_cfg<F, 1, 4, 1, 1, DUAL>(p, st);
    if (p.M <= 64) return launch_cfg<F, 2, 2, 1, 1, DUAL>(p, st);
    if (p.M <= 512) return launch_cfg<F, 2, 2, 2, 2, DUAL>(p, st);
    return launch_cfg<F, 2, 2, 4, 2, DUAL>(p, st);
}

hipError_t launch_gemm(const GemmParams& p, hipStream_t st) {
    const bool dual = p.W2 != nullptr;
    switch (p.format) {
        case QUANT_Q4_0: return dual ? launch_fmt<QUANT_Q4_0, true>(p, st) : launch_fmt<QUANT_Q4_0, false>(p, st);
        case QUANT_MLX_4BIT: return dual ? launch_fmt<QUANT_MLX_4BIT, true>(p, st) : launch_fmt<QUANT_MLX_4BIT, false>(p, st);
        case QUANT_Q4_K: return dual ? launch_fmt<QUANT_Q4_K, true>(p, st) : launch_fmt<QUANT_Q4_K, false>(p, st);
        case QUANT_TERNARY_1_58: return dual ? launch_fmt<QUANT_TERNARY_1_58, true>(p, st) : launch_fmt<QUANT_TERNARY_1_58, false>(p, st);
        default: return hipErrorInvalidValue;
    }
}

// --------------------------------------------------------------------------
// Dequantize [N, K] weights to binary16 with the same decoders the GEMM uses
// (bit-exact contract check; also the reference registry's dequantize hook,
// src/router/quant_registry.h:24).  One thread per 32-element group.
// --------------------------------------------------------------------------
template <int F>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* W, _Float16* out, uint32_t K, uint32_t N,
                                                      uint32_t col_bytes) {
    using Dec = Decoder<F>;
    const uint32_t ng = K / 32;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)ng * N) return;
    const uint32_t n = (uint32_t)(idx / ng), g = (uint32_t)(idx % ng);
    // Base at the (4-byte aligned) start of W; the column offset carries the
    // 2-byte parity of 18-byte Q4_0 columns.
    auto r = make_rsrc(W, (uint32_t)((size_t)col_bytes * N));
    uint32_t raw[Dec::kRawWords], o[16];
    Dec::load(r, n * col_bytes, g, raw);
    Dec::decode(raw, Dec::parity(n * col_bytes, g), o);
    u4_t* dst = reinterpret_cast<u4_t*>(out + (size_t)n * K + (size_t)g * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) dst[j] = u4_t{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
}

hipError_t launch_dequant(int format, const uint8_t* W, _Float16* out, uint32_t K, uint32_t N, size_t col_bytes,
                          hipStream_t st) {
    const size_t total = (size_t)(K / 32) * N;
    dim3 grid((unsigned)((total + 255) / 256));
    switch (format) {
        case QUANT_Q4_0: hipLaunchKernelGGL(dequant_kernel<QUANT_Q4_0>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_MLX_4BIT: hipLaunchKernelGGL(dequant_kernel<QUANT_MLX_4BIT>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_Q4_K: hipLaunchKernelGGL(dequant_kernel<QUANT_Q4_K>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_TERNARY_1_58: hipLaunchKernelGGL(dequant_kernel<QUANT_TERNARY_1_58>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qr
