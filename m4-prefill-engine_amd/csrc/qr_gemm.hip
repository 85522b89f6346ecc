// qr_gemm.hip -- quantized projection Y = X . W^T on gfx950 MFMA (tiled, M > 64).
//
// Replaces the reference's block_mma_64x64_engine (quant_router_kernels.metal:
// 442-581) and its 14 entry points (:588-927), and the fused dual-projection
// SwiGLU swiglu_mma_dual_simd (brick3_swiglu_kernels.metal:428-698).
//
// Design (one workgroup = 4 or 8 wave64s, one BM x BN output tile, the K range
// split across `ksplit` workgroups when the tile grid alone cannot fill the GPU):
//  * K advances 64 per step (two 32-element weight groups per column).
//  * The X tile [BM x 64] fp16 is fetched with 16-byte buffer loads; the
//    weight groups of the BN columns are fetched raw (compressed) and decoded
//    in registers to binary16 (qr_decode.h, bit-exact vs the CPU unpack), a
//    half group (16 elements) per thread when the workgroup has enough threads.
//    Fetches run P steps ahead of the MFMAs (P register stages), so HBM/L2
//    latency hides behind P-1 steps of matrix work.
//  * Decoded tiles go to a double-buffered LDS stage (one barrier per step).
//    Both operands are K-contiguous, so each lane fetches its 8 halfs of a
//    v_mfma_f32_32x32x16_f16 operand with one ds_read_b128; rows are padded
//    by 8 halfs to spread the LDS banks.  With 8 waves, two waves share each
//    SIMD, so one wave's decode VALU work overlaps the other's MFMAs.
//  * Tiles are assigned XCD-aware: consecutive workgroup ids land on
//    different XCDs, so ids are remapped to give each XCD a contiguous run of
//    tiles grouped 2 row-tiles x many column-tiles (shared L2 reuse of X
//    rows and weight columns).
//  * Epilogue: fp32 accumulators (+ fp16 residual, + SwiGLU for the dual
//    variant) rounded once to fp16, written [M, N] or head-major [H, M, D]
//    (quant_router_kernels.metal:570-574).  With a K split, the partial
//    accumulators go to a workspace with agent-scope stores and the last
//    workgroup of the tile (agent-scope counter) sums them in split order --
//    deterministic, one launch.
#include "qr_decode.h"
#include "qr_kernels.h"

#include <stdlib.h>

namespace qr {

constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;  // halfs per LDS row (padding vs bank conflicts)

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL>
struct GemmCfg {
    static constexpr int NT = 64 * WGM * WGN;             // threads
    static constexpr int BM = WGM * TM * 32;
    static constexpr int BN = WGN * TN * 32;
    static constexpr int NCOL = DUAL ? 2 * BN : BN;       // weight columns decoded per step
    static constexpr int HALVES = NCOL * 4;               // 16-element half groups per step
    static constexpr bool HALF = NT >= HALVES;            // one half group per thread
    static constexpr int UNITS = HALF ? HALVES : NCOL * 2;
    static constexpr int UPT = (UNITS + NT - 1) / NT;     // decode units per thread
    static constexpr int XCH = BM * kBK / 8;              // 16-byte X chunks per step
    static constexpr int XPT = (XCH + NT - 1) / NT;
    static constexpr int LDS_A = BM * kLdsRow;            // halfs per stage
    static constexpr int LDS_B = NCOL * kLdsRow;
    static constexpr int LDS_STAGE = LDS_A + LDS_B;
    static constexpr int ACC = TM * TN * 16 * (DUAL ? 2 : 1);  // accumulator floats per lane
    static_assert(WGM * WGN == 4 || WGM * WGN == 8, "4 or 8 waves per workgroup");
};

// Tile of workgroup `bid` among T tiles (nt_m x nt_n): XCD-contiguous runs,
// grouped two row-tiles at a time.
__device__ __forceinline__ void tile_of(uint32_t bid, uint32_t nt_m, uint32_t nt_n, uint32_t& tm, uint32_t& tn) {
    const uint32_t T = nt_m * nt_n;
    uint32_t t = bid;
    if (T % 8 == 0) t = (bid % 8) * (T / 8) + bid / 8;
    constexpr uint32_t GM = 2;
    const uint32_t per_group = GM * nt_n;
    const uint32_t grp = t / per_group;
    const uint32_t first = grp * GM;
    const uint32_t gm = min(GM, nt_m - first);
    const uint32_t in = t % per_group;
    tm = first + in % gm;
    tn = in / gm;
}

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL, int P>
__global__ void __launch_bounds__(64 * WGM * WGN)
gemm_kernel(GemmParams p) {
    using C = GemmCfg<F, WGM, WGN, TM, TN, DUAL>;
    using Dec = Decoder<F>;
    constexpr int NT = C::NT;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nt_m = (M + C::BM - 1) / C::BM, nt_n = (N + C::BN - 1) / C::BN;
    uint32_t tmi, tni;
    tile_of(blockIdx.x, nt_m, nt_n, tmi, tni);
    const int m0 = tmi * C::BM, n0 = tni * C::BN;
    const uint32_t ksplit = p.ksplit ? p.ksplit : 1;
    const uint32_t kz = blockIdx.y;
    const uint32_t Kc = K / ksplit;                        // host guarantees divisibility
    const uint32_t k_begin = kz * Kc;
    const uint32_t nsteps = (Kc + kBK - 1) / kBK;
    const uint32_t g_begin = k_begin / 32, g_end = (k_begin + Kc) / 32;
    const uint32_t col_bytes = (uint32_t)p.col_bytes;

    const int mrows = min(C::BM, (int)M - m0);
    const int ncols = min(C::BN, (int)N - n0);
    auto xr = make_rsrc(p.X + (size_t)m0 * K, (uint32_t)mrows * K * 2u);
    auto wr0 = make_rsrc(p.W + (size_t)n0 * col_bytes, (uint32_t)ncols * col_bytes);
    auto wr1 = make_rsrc(DUAL ? p.W2 + (size_t)n0 * col_bytes : p.W, DUAL ? (uint32_t)ncols * col_bytes : 0u);

    uint32_t xraw[P][C::XPT][4];
    uint32_t wraw[P][C::UPT][Dec::kRawWords];

    // decode unit u of this thread: weight column, group within the step, half
    auto unit_of = [&](int u, int& col, int& gsel, int& half) {
        const int unit = tid + NT * u;
        if (C::HALF) {
            col = unit >> 2;
            gsel = (unit >> 1) & 1;
            half = unit & 1;
        } else {
            col = unit >> 1;
            gsel = unit & 1;
            half = -1;
        }
    };

    auto load_step = [&](uint32_t step, int slot) {
        const uint32_t k0 = k_begin + step * kBK;
#pragma unroll
        for (int i = 0; i < C::XPT; i++) {
            const int c = tid + NT * i;
            const int row = c >> 3, kc = c & 7;
            const uint32_t k = k0 + kc * 8;
            const uint32_t off = (c < C::XCH && k < k_begin + Kc) ? ((uint32_t)row * K + k) * 2u : kOOB;
            const u4_t v = ld_b128(xr, off);
            xraw[slot][i][0] = v.x; xraw[slot][i][1] = v.y; xraw[slot][i][2] = v.z; xraw[slot][i][3] = v.w;
        }
#pragma unroll
        for (int u = 0; u < C::UPT; u++) {
            int col, gsel, half;
            unit_of(u, col, gsel, half);
            const uint32_t g = g_begin + step * 2 + gsel;
            const bool up = DUAL && col >= C::BN;
            const int lcol = up ? col - C::BN : col;
            // out-of-range groups read as zeros (buffer bounds) and decode to zeros
            const uint32_t coff = ((C::UNITS % NT == 0 || tid + NT * u < C::UNITS) && g < g_end) ? (uint32_t)lcol * col_bytes : kOOB;
            Dec::load(up ? wr1 : wr0, coff, coff == kOOB ? 0u : g, wraw[slot][u]);
        }
    };

    auto store_step = [&](uint32_t step, int slot, int stage) {
        _Float16* As = lds + stage * C::LDS_STAGE;
        _Float16* Bs = As + C::LDS_A;
#pragma unroll
        for (int i = 0; i < C::XPT; i++) {
            const int c = tid + NT * i;
            if (C::XCH % NT == 0 || c < C::XCH) {
                const int row = c >> 3, kc = c & 7;
                *reinterpret_cast<u4_t*>(As + row * kLdsRow + kc * 8) =
                    u4_t{xraw[slot][i][0], xraw[slot][i][1], xraw[slot][i][2], xraw[slot][i][3]};
            }
        }
#pragma unroll
        for (int u = 0; u < C::UPT; u++) {
            if (C::UNITS % NT == 0 || tid + NT * u < C::UNITS) {
                int col, gsel, half;
                unit_of(u, col, gsel, half);
                const uint32_t g = g_begin + step * 2 + gsel;
                const int lcol = (DUAL && col >= C::BN) ? col - C::BN : col;
                const uint32_t par = Dec::parity((uint32_t)lcol * col_bytes, g);
                if (C::HALF) {
                    uint32_t out[8];
                    Dec::decode_half(wraw[slot][u], par, half, out);
                    u4_t* dst = reinterpret_cast<u4_t*>(Bs + col * kLdsRow + gsel * 32 + half * 16);
                    dst[0] = u4_t{out[0], out[1], out[2], out[3]};
                    dst[1] = u4_t{out[4], out[5], out[6], out[7]};
                } else {
                    uint32_t out[16];
                    decode_group<F>(wraw[slot][u], par, out);
                    u4_t* dst = reinterpret_cast<u4_t*>(Bs + col * kLdsRow + gsel * 32);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        dst[j] = u4_t{out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]};
                }
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

    const int arow = wm * TM * 32 + (lane & 31);
    const int bcol = wn * TN * 32 + (lane & 31);
    const int kq = (lane >> 5) * 8;

    auto compute = [&](int stage) {
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
    };

    // ---- prologue: fill the P register stages, stage step 0 into LDS ----
#pragma unroll
    for (int j = 0; j < P; j++)
        if ((uint32_t)j < nsteps) load_step(j, j);
    store_step(0, 0, 0);
    if ((uint32_t)P < nsteps) load_step(P, 0);
    __syncthreads();

    // ---- main loop, unrolled by P so register stages are static.  Full groups
    // of P steps run branch-free (the last group's look-ahead fetches fall out
    // of range and read zeros), so the MFMAs of step s, the decode and LDS
    // stores of step s+1 and the fetches of step s+1+P form one basic block
    // that the scheduler interleaves. ----
    uint32_t s0 = 0;
    for (; s0 + P <= nsteps; s0 += P) {
#pragma unroll
        for (int j = 0; j < P; j++) {
            const uint32_t s = s0 + j;
            const int slot = (j + 1) % P;
            compute(s & 1);
            store_step(s + 1, slot, (s + 1) & 1);
            load_step(s + 1 + P, slot);
            __syncthreads();
        }
    }
#pragma unroll
    for (int j = 0; j < P; j++) {
        const uint32_t s = s0 + j;
        if (s < nsteps) {
            compute(s & 1);
            if (s + 1 < nsteps) {
                const int slot = (j + 1) % P;
                store_step(s + 1, slot, (s + 1) & 1);
                if (s + 1 + P < nsteps) load_step(s + 1 + P, slot);
            }
            __syncthreads();
        }
    }

    // ---- split-K: publish partials, the last workgroup of the tile sums ----
    if (ksplit > 1) {
        const uint32_t T = nt_m * nt_n;
        const uint32_t tile = tmi * nt_n + tni;
        float* slot = p.ws + ((size_t)kz * T + tile) * (C::ACC * NT) + tid;
        int e = 0;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++, e++) {
                    __hip_atomic_store(slot + e * NT, acc[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if constexpr (DUAL)
                        __hip_atomic_store(slot + (C::ACC / 2 + e) * NT, acc2[i][j][r], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores performed
        __syncthreads();
        __shared__ uint32_t s_last;
        if (tid == 0) {
            const uint32_t prev =
                __hip_atomic_fetch_add(p.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = (prev == ksplit - 1) ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        // sum all splits in split order (deterministic)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                acc[i][j] = f16v_t{};
                if constexpr (DUAL) acc2[i][j] = f16v_t{};
            }
        for (uint32_t z = 0; z < ksplit; z++) {
            const float* src = p.ws + ((size_t)z * T + tile) * (C::ACC * NT) + tid;
            int e2 = 0;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++, e2++) {
                        acc[i][j][r] += __hip_atomic_load(src + e2 * NT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if constexpr (DUAL)
                            acc2[i][j][r] += __hip_atomic_load(src + (C::ACC / 2 + e2) * NT, __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
                    }
        }
        if (tid == 0) __hip_atomic_store(p.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- epilogue: accumulator element r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
    // column l%32 of the 32x32 MFMA tile.  The (SwiGLU-combined) fp32 values go
    // through LDS, one 32-row band of the wave tile at a time, so that each
    // lane then owns 8 consecutive columns of one row: the residual is read and
    // the output written with 16-byte accesses, and the value is rounded to
    // fp16 once, after the residual add. ----
    auto value = [&](int i, int j, int r) {
        float v = acc[i][j][r];
        if constexpr (DUAL) {
            const float u = acc2[i][j][r];
            v = v / (1.0f + __expf(-v)) * u;
        }
        return v;
    };
    const bool vec_io = ((reinterpret_cast<uintptr_t>(p.Y) | reinterpret_cast<uintptr_t>(p.R)) & 15u) == 0 &&
                        (N & 7u) == 0 && (p.head_D & 7u) == 0;
    if (vec_io) {
        constexpr int WC = TN * 32;        // wave tile columns
        constexpr int ERS = WC + 4;        // padded LDS row (floats)
        static_assert(WGM * WGN * 32 * ERS * 4 <= 2 * C::LDS_STAGE * 2, "epilogue staging fits the LDS stages");
        float* E = reinterpret_cast<float*>(lds) + wave * 32 * ERS;
        __syncthreads();  // every wave is done with the operand stages
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    E[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * ERS + j * 32 + (lane & 31)] = value(i, j, r);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS writes done (wave-local region)
            __builtin_amdgcn_wave_barrier();
            constexpr int CHUNKS = 32 * WC / 8;  // 8-column chunks in the band
#pragma unroll
            for (int c = lane; c < CHUNKS; c += 64) {
                const int row = c / (WC / 8), c8 = c % (WC / 8);
                const int m = m0 + wm * TM * 32 + i * 32 + row;
                const int n = n0 + wn * WC + c8 * 8;
                if (m < (int)M && n < (int)N) {
                    const f4_t lo = *reinterpret_cast<const f4_t*>(E + row * ERS + c8 * 8);
                    const f4_t hi = *reinterpret_cast<const f4_t*>(E + row * ERS + c8 * 8 + 4);
                    float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    if (p.R) {
                        const u4_t rr = *reinterpret_cast<const u4_t*>(p.R + (size_t)m * N + n);
                        const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const h2_t h = as_h2(rw[q]);
                            v[2 * q] += (float)h.x;
                            v[2 * q + 1] += (float)h.y;
                        }
                    }
                    u4_t o;
                    o.x = pack_h2(f2h_bits(v[0]), f2h_bits(v[1]));
                    o.y = pack_h2(f2h_bits(v[2]), f2h_bits(v[3]));
                    o.z = pack_h2(f2h_bits(v[4]), f2h_bits(v[5]));
                    o.w = pack_h2(f2h_bits(v[6]), f2h_bits(v[7]));
                    size_t off;
                    if (p.head_D) {
                        const uint32_t h = (uint32_t)n / p.head_D, dd = (uint32_t)n % p.head_D;
                        off = ((size_t)h * M + m) * p.head_D + dd;
                    } else {
                        off = (size_t)m * N + n;
                    }
                    *reinterpret_cast<u4_t*>(p.Y + off) = o;
                }
            }
            __builtin_amdgcn_wave_barrier();  // band reads done before the next band overwrites
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * TN * 32 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * TM * 32 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < (int)M && n < (int)N) {
                    float v = value(i, j, r);
                    if (p.R) v += (float)p.R[(size_t)m * N + n];
                    size_t o;
                    if (p.head_D) {
                        const uint32_t h = (uint32_t)n / p.head_D, dd = (uint32_t)n % p.head_D;
                        o = ((size_t)h * M + m) * p.head_D + dd;
                    } else {
                        o = (size_t)m * N + n;
                    }
                    p.Y[o] = (_Float16)v;
                }
            }
        }
}

#ifndef QR_GEMM_STAGES
#define QR_GEMM_STAGES 3
#endif

// Tile configurations: {waves_m, waves_n, tiles_m, tiles_n} -> BM x BN.
//   0: 8 waves 4x2, 2x2 tiles -> 256 x 128  (large M)
//   1: 4 waves 2x2, 2x2 tiles -> 128 x 128  (medium M)
//   2: 4 waves 2x2, 1x2 tiles ->  64 x 128
//   dual (SwiGLU): 3: 8 waves 4x2, 2x1 -> 256 x 64 (gate + up: 128 weight
//   columns per step); 4: 4 waves 2x2, 1x1 -> 64 x 64
static int pick_shape(uint32_t M, bool dual) {
    if (dual) return M > 64 ? 3 : 4;
    if (M >= 1024) return 0;
    if (M > 64) return 1;
    return 2;
}

static void shape_dims(int shape, uint32_t& bm, uint32_t& bn) {
    switch (shape) {
        case 0: bm = 256; bn = 128; return;
        case 1: bm = 128; bn = 128; return;
        case 2: bm = 64; bn = 128; return;
        case 3: bm = 256; bn = 64; return;
        default: bm = 64; bn = 64; return;
    }
}

template <int F, int WGM, int WGN, int TM, int TN, bool DUAL>
static hipError_t launch_cfg(const GemmParams& p, hipStream_t st) {
    using C = GemmCfg<F, WGM, WGN, TM, TN, DUAL>;
    auto kern = gemm_kernel<F, WGM, WGN, TM, TN, DUAL, QR_GEMM_STAGES>;
    const size_t lds = 2 * C::LDS_STAGE * sizeof(_Float16);
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t T = ((p.M + C::BM - 1) / C::BM) * ((p.N + C::BN - 1) / C::BN);
    const uint32_t ks = p.ksplit ? p.ksplit : 1;
    hipLaunchKernelGGL(kern, dim3(T, ks), dim3(C::NT), lds, st, p);
    return hipGetLastError();
}

// Kernel selection: the register-B kernel (qr_gemm_rb.hip) unless
// QR_GEMM_IMPL=lds selects the LDS-staged one.
static bool use_rb() {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("QR_GEMM_IMPL");
        v = (e && e[0] == 'l') ? 0 : 1;
    }
    return v == 1;
}

uint32_t gemm_pick_ksplit(const GemmParams& p) {
    if (use_rb()) return gemm_rb_pick_ksplit(p);
    const bool dual = p.W2 != nullptr;
    if (dual) return 1;
    uint32_t bm, bn;
    shape_dims(pick_shape(p.M, dual), bm, bn);
    const uint32_t T = ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
    uint32_t ks = 1;
    // split K until the grid covers the 256 CUs; each split keeps >= 1024 of K
    // and a whole number of 256-element super-blocks
    while (T * ks < 256 && p.K % (256 * ks * 2) == 0 && p.K / (ks * 2) >= 1024) ks *= 2;
    return ks;
}

size_t gemm_workspace_floats(const GemmParams& p, uint32_t ks, uint32_t* tiles) {
    if (use_rb()) return gemm_rb_workspace_floats(p, ks, tiles);
    uint32_t bm, bn;
    const bool dual = p.W2 != nullptr;
    shape_dims(pick_shape(p.M, dual), bm, bn);
    const uint32_t T = ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
    if (tiles) *tiles = T;
    return ks > 1 ? (size_t)ks * T * bm * bn * (dual ? 2 : 1) : 0;
}

template <int F, bool DUAL>
static hipError_t launch_fmt(const GemmParams& p, hipStream_t st) {
    if constexpr (DUAL) {
#ifndef QR_DUAL_CFG
#define QR_DUAL_CFG 2
#endif
        if (pick_shape(p.M, true) == 3) {
            if (QR_DUAL_CFG == 1) return launch_cfg<F, 2, 2, 2, 1, true>(p, st);
            if (QR_DUAL_CFG == 2) return launch_cfg<F, 4, 2, 2, 1, true>(p, st);
            if (QR_DUAL_CFG == 3) return launch_cfg<F, 2, 2, 2, 2, true>(p, st);
            return launch_cfg<F, 4, 2, 1, 1, true>(p, st);
        }
        return launch_cfg<F, 2, 2, 1, 1, true>(p, st);
    } else {
        switch (pick_shape(p.M, false)) {
            case 0: return launch_cfg<F, 4, 2, 2, 2, false>(p, st);
            case 1: return launch_cfg<F, 2, 2, 2, 2, false>(p, st);
            default: return launch_cfg<F, 2, 2, 1, 2, false>(p, st);
        }
    }
}

hipError_t launch_gemm(const GemmParams& p0, hipStream_t st) {
    if (use_rb()) {
        GemmParams p = p0;
        p.group_m = gemm_rb_group_m(p);
        return launch_gemm_rb(p, st);
    }
    const GemmParams& p = p0;
    const bool dual = p.W2 != nullptr;
    switch (p.format) {
        case QUANT_Q4_0: return dual ? launch_fmt<QUANT_Q4_0, true>(p, st) : launch_fmt<QUANT_Q4_0, false>(p, st);
        case QUANT_MLX_4BIT: return dual ? launch_fmt<QUANT_MLX_4BIT, true>(p, st) : launch_fmt<QUANT_MLX_4BIT, false>(p, st);
        case QUANT_Q4_K: return dual ? launch_fmt<QUANT_Q4_K, true>(p, st) : launch_fmt<QUANT_Q4_K, false>(p, st);
        case QUANT_TERNARY_1_58: return dual ? launch_fmt<QUANT_TERNARY_1_58, true>(p, st) : launch_fmt<QUANT_TERNARY_1_58, false>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qr
