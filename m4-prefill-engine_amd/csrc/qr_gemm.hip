// qr_gemm.hip -- quantized projection Y = X . W^T on gfx950 MFMA, weights
// decoded straight into MFMA B-operand registers (tiled, M > 64).
// Built once per format with -DQR_GEMM_FORMAT=F (one kernel family per
// compilation unit, so the formats compile in parallel).
//
// Replaces the reference's block_mma_64x64_engine (quant_router_kernels.metal:
// 442-581) with its entry points (:588-927), and the fused dual-projection
// SwiGLU swiglu_mma_dual_simd (brick3_swiglu_kernels.metal:428-698).
//
// One workgroup = NW wave64s and one BM x BN output tile, the waves arranged
// as WR row groups x NW / WR column groups of 32 TM x 32 TN wave tiles.  With
// WR = 1 every weight column belongs to exactly one wave and is decoded
// exactly once per workgroup; WR = 2 decodes each column in two waves (one
// per row group) for twice the waves per SIMD at the same tile:
//  * K advances 64 per step = two 32-element quant groups per column.  For
//    v_mfma_f32_32x32x16_f16 lane l supplies column l % 32 and the 8 k values
//    8 (l / 32) .. +7 of each 16-wide slice; here the K order inside a step is
//    permuted so that lane half h = l / 32 owns quant group h of the step
//    whole: at slice kk the lane holds elements 8 kk .. 8 kk + 7 of its group.
//    The sum over k is order-free, so X (the A operand) is read with the same
//    permutation: row r, k = 32 h + 8 kk + i.
//  * Each lane fetches the raw block of its (column, group) with buffer loads
//    P steps ahead and decodes all 32 weights to binary16 in registers
//    (qr_decode.h: bit-exact vs the CPU unpack).  No LDS traffic for weights.
//  * The X tile [BM x 64] fp16 is fetched with 16-byte buffer loads (P steps
//    ahead) into a double-buffered LDS stage, padded 8 halfs per row so the
//    ds_read_b128 fragment reads are bank-conflict free; one barrier per step.
//    Per step a wave reads BM x 64 x 2 bytes of LDS for BM x 32 TN x 64 x 2
//    flop: with TN = 2 that is half the LDS bandwidth at full MFMA rate.
//  * The MFMAs of step s, the decode of step s + 1 and the fetches of step
//    s + 1 + P sit in one basic block (the main loop is unrolled by P and
//    branch-free), so decode VALU work issues under the matrix pipe.
//  * XCD-aware tile order (consecutive workgroup ids land on different XCDs):
//    each XCD gets a contiguous run of tiles, grouped GM row-tiles x many
//    column-tiles so X rows and weight columns are reused from its L2.
//  * Epilogue: fp32 accumulators (+ fp16 residual, + SwiGLU for the dual
//    variant) rounded once to fp16, staged through LDS for 16-byte stores,
//    written [M, N] or head-major [H, M, D] (quant_router_kernels.metal:570-574).
//    K split across workgroups: each split writes fp32 partials to a
//    workspace and a second, elementwise kernel sums them in split order and
//    runs the same epilogue -- deterministic, ordered by the kernel boundary.
#include "qr_decode.h"
#include "qr_gemm_shapes.h"

namespace qr {


namespace rb {

constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;  // halfs per LDS row of the X stage

// Whether an instance stages X through a stager wave: one 32-column tile per
// wave and no SwiGLU pair (the instances that leave registers for the extra
// wave), except Q4_K's 8-wave tile, whose registers then spill for no gain.
constexpr bool use_stager(int F, int TN, int NW, int KG, bool DUAL) {
    return !DUAL && TN == 1 && !(F == QUANT_Q4_K && NW == 8 && KG == 1);
}

// Weights through the stager too (WST): the K-group tiles with MLX blocks
// (20 bytes per group: one round of two 64-K steps is 80 bytes, 5 whole
// 16-byte units, per column).  The stager copies each round's weights into a
// 4-stage LDS ring ahead of the round's X; the compute waves read their raw
// words from LDS just before decoding instead of fetching them (headline
// 32.1 -> 31.3 us over four rounds).
constexpr bool use_wstage(int F, int KG, bool stager) {
    return stager && KG == 2 && F == QUANT_MLX_4BIT;
}
constexpr int kWRoundBytes = 80;  // one column's weights of one round (MLX)
constexpr int kWStages = 4;

// NW waves as KG K groups of WR row groups x NW / (WR KG) column groups; a
// wave's tile is 32 TM rows x 32 TN columns.  With KG = 2 the groups take
// alternate K steps of the whole K range and sum their tiles in LDS at the end.
template <int TM, int TN, int NW, int WR, int KG, bool DUAL, bool STAGER>
struct Cfg {
    static_assert(NW % (WR * KG) == 0, "whole column groups");
    static constexpr int NT = 64 * NW;
    static constexpr int WC = NW / (WR * KG);     // column groups
    static constexpr int WM = 32 * TM;            // rows per wave
    static constexpr int BM = WR * WM;
    static constexpr int WN = 32 * TN;            // columns per wave
    static constexpr int BN = WC * WN;
    static constexpr int NCB = DUAL ? 2 * TN : TN;  // 32-column B tiles per wave (gate, then up)
    static constexpr int XCH = BM * kBK / 8;      // 16-byte X chunks per step
    static constexpr int XPT = (XCH + NT - 1) / NT;
    // stager stages: unpadded, XOR-swizzled rows (the lane's 4 TM read offsets
    // held in registers), except where two 128-row waves per SIMD leave no
    // registers for them (the 8-wave 128 x 256 tile then spills: ternary at
    // M = 2048 80 vs 69 us); there the rows keep their pad unit
    static constexpr bool XSW = STAGER && (NW == 4 || TM <= 2);
    static constexpr int XROW = XSW ? kBK : kLdsRow;  // halfs per LDS row of an X stage
    static constexpr int LDS_STAGE = BM * XROW;   // halfs
    // X staging: an extra stager wave copies X to LDS (XST: KG (XD + 1)
    // stages, XD rounds ahead), or every wave fetches X into registers and
    // writes it to a 3-stage ring.
    static constexpr bool XST = STAGER;
    static constexpr int NTL = NT + (XST ? 64 : 0);  // threads per workgroup
    static_assert(KG == 1 || XST, "K groups take X from the stager");
    static constexpr int XD = KG > 1 ? 3 : 5;                // rounds of KG steps the copies run ahead
    static constexpr int XS = XST ? KG * (XD + 1) : 3;       // X stages in LDS
    static constexpr int U = KG > 1 ? 4 : 6;                 // rounds unrolled (ring indices static)
    static constexpr int XCP = BM * (XROW / 8) / 64;  // 64-lane copies per stage
    static constexpr int ACC = TM * NCB * 16;     // accumulator floats per lane
    // Epilogue staging (floats): the 32-column tile j of a wave row starts at
    // column EJS * j and rows are ERS apart.  The compiler pairs the band's
    // LDS writes across tiles (TN > 1) or across rows (TN == 1); a pair
    // distance of 16 (mod 32) words puts a lane's two dwords in opposite bank
    // halves.  The row distances also keep the 16-byte reads conflict free
    // whether a read pass serves 8 lanes from 32 banks or 16 lanes from 64.
    static constexpr int EJS = TN > 1 ? 48 : 32;
    static constexpr int ERS = TN > 1 ? (EJS * (TN - 1) + 32 + 31) / 32 * 32 : 48;
    static constexpr int EPI_BYTES = NW * 32 * ERS * 4;
    static constexpr int KGX_BYTES = KG > 1 ? NW / KG * ACC * 64 * 4 : 0;  // K-group exchange
    static constexpr int LDS_BYTES0 = XS * LDS_STAGE * 2 > EPI_BYTES ? XS * LDS_STAGE * 2 : EPI_BYTES;
    static constexpr int LDS_BYTES = LDS_BYTES0 > KGX_BYTES ? LDS_BYTES0 : KGX_BYTES;
};

// Swizzle of the stager's unpadded 128-byte X rows: logical 16-byte unit c of
// row r sits at unit c ^ xswz(r).  The 8 rows of one ds_read_b128 pass (and
// the 16 rows of a pass that serves 16 lanes from 64 banks: rows of one parity
// take the even or the odd values) hit distinct bank groups.
__device__ __forceinline__ uint32_t xswz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

__device__ __forceinline__ void tile_of(uint32_t bid, uint32_t nt_m, uint32_t nt_n, uint32_t gm_req, uint32_t& tm,
                                        uint32_t& tn) {
    const uint32_t T = nt_m * nt_n;
    uint32_t t = bid;
    if (T % 8 == 0) t = (bid % 8) * (T / 8) + bid / 8;
    const uint32_t GM = gm_req ? gm_req : 2;
    const uint32_t per_group = GM * nt_n;
    const uint32_t grp = t / per_group;
    const uint32_t first = grp * GM;
    const uint32_t gm = min(GM, nt_m - first);
    const uint32_t in = t % per_group;
    tm = first + in % gm;
    tn = in / gm;
}

}  // namespace rb

// SPLIT: the instance writes split-K partials (the stores are compiled only
// into the instances that split).  P: weight fetch distance in steps.
// kVpm: VALU ops scheduled beside each MFMA of a k-slice (kVpmKG in the
// K-group tiles, whose decode is their only VALU work in the loop: headline
// 31.2 -> 30.5 us with 3 instead of 5, four paired rounds).
constexpr int kWeightStages = 2;
constexpr int kVpm = 5;
constexpr int kVpmKG = 3;
// s_waitcnt vmcnt(N), N an immediate.
template <uint32_t N>
__device__ __forceinline__ void rb_wait_vmcnt() {
    static_assert(N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int F, int TM, int TN, int NW, int WR, int KG, bool DUAL, int P, bool SPLIT>
__global__ void __launch_bounds__(64 * NW + (rb::use_stager(F, TN, NW, KG, DUAL) ? 64 : 0), 1)
gemm_rb_kernel(GemmParams p) {
    using C = rb::Cfg<TM, TN, NW, WR, KG, DUAL, rb::use_stager(F, TN, NW, KG, DUAL)>;
    static_assert(!(SPLIT && KG > 1), "K groups replace the K split");
    constexpr bool WST = rb::use_wstage(F, KG, C::XST);
    constexpr int WRING = WST ? rb::kWStages * C::BN * rb::kWRoundBytes : 0;  // bytes
    constexpr int XBYTES = C::XS * C::LDS_STAGE * 2;                           // X stages (bytes)
    static_assert(!WST || C::BN * rb::kWRoundBytes % 1024 == 0, "whole 1 KB weight copies per round");
    using Dec = Decoder<F>;
    constexpr int NT = C::NT;
    constexpr int NCB = C::NCB;
    constexpr int kBK = rb::kBK;
    constexpr int kLdsRow = rb::kLdsRow;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    const int kg = KG > 1 ? wave / (NW / KG) : 0, wl = KG > 1 ? wave % (NW / KG) : wave;  // K group, wave in it
    const int wrow = wl / C::WC, wcolg = wl % C::WC;       // this wave's row group and column group
    const int h = lane >> 5;     // quant group of the step this lane owns
    const int c32 = lane & 31;

    // grouped launch: the group of this workgroup's tile takes over W / Y / N
    uint32_t bid = blockIdx.x;
    if (p.ngroups > 1) {
        const uint32_t ntm = (p.M + C::BM - 1) / C::BM;
        const uint32_t t0 = ntm * ((p.N + C::BN - 1) / C::BN);
        if (bid >= t0) {
            bid -= t0;
            const uint32_t t1 = ntm * ((p.Nx[0] + C::BN - 1) / C::BN);
            const int gx = (bid < t1 || p.ngroups == 2) ? 0 : 1;
            if (gx == 1) bid -= t1;
            p.W = p.Wx[gx];
            p.Y = p.Yx[gx];
            p.N = p.Nx[gx];
        }
    }
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nt_m = (M + C::BM - 1) / C::BM, nt_n = (N + C::BN - 1) / C::BN;
    uint32_t tmi, tni;
    rb::tile_of(bid, nt_m, nt_n, p.group_m, tmi, tni);
    const int m0 = tmi * C::BM, n0 = tni * C::BN;
    const uint32_t ksplit = p.ksplit ? p.ksplit : 1;
    const uint32_t kz = blockIdx.y;
    const uint32_t Kc = K / ksplit;  // host guarantees divisibility (and Kc % 32 == 0)
    const uint32_t k_begin = kz * Kc, k_end = k_begin + Kc;
    const uint32_t nsteps = (Kc + kBK - 1) / kBK;
    const uint32_t g_begin = k_begin / 32, g_end = k_end / 32;
    const uint32_t col_bytes = (uint32_t)p.col_bytes;

    const int mrows = min(C::BM, (int)M - m0);
    const int ncols = min(C::BN, (int)N - n0);
    auto xr = make_rsrc(p.X + (size_t)m0 * K, (uint32_t)mrows * K * 2u);
    // ---- X stager (XST): the extra wave NW copies each step's BM x 64 slice of X
    // into an LDS stage (XSW: 128-byte rows, units XOR-swizzled; else rows of
    // kLdsRow halfs: 8 16-byte units and a pad unit, copied as zeros) by
    // buffer-load-to-LDS, XD steps ahead, through
    // a ring of XS stages; the compute waves never touch X in memory.  Before
    // the barrier that opens step t it waits (its own copies, in order) for
    // the copies of step t + 1, whose first k-slice the compute waves read
    // during step t; after it, stage (t + XD) % XS = (t - 1) % XS is free. It
    // leaves after the barrier of the last step (a finished wave no longer
    // holds barriers).  With K groups a round is KG consecutive steps, one
    // per group, and the same holds per round. ----
    if (C::XST && wave == NW) {
        // raised wave priority: on the SIMD it shares with a compute wave, the
        // stager's copies and waits issue ahead of that wave's MFMA / VALU
        // stream (headline 31.3 -> 30.1 us over five paired rounds)
        __builtin_amdgcn_s_setprio(2);
        uint32_t xo[C::XCP], xh[C::XCP];  // per-lane offsets: whole step, first half (a 32-K last step)
#pragma unroll
        for (int q = 0; q < C::XCP; q++) {
            uint32_t row, cu;
            bool live;
            if constexpr (C::XSW) {  // LDS unit pu of a row holds logical unit pu ^ xswz(row)
                const uint32_t u = 64u * q + lane;
                row = u / 8u;
                cu = (u % 8u) ^ rb::xswz(row);
                live = true;
            } else {  // 9 units per row, the ninth a pad copied as zeros
                const uint32_t u = 64u * q + lane;
                row = u / 9u;
                cu = u % 9u;
                live = cu < 8;
            }
            xo[q] = live && row < (uint32_t)mrows ? (row * K + 8u * cu) * 2u : kOOB;
            xh[q] = cu < 4 ? xo[q] : kOOB;
        }
        // weight copies of a round (WST): LDS unit u = col * 5 + unit of the
        // stage, copy c covering units 64 c .. 64 c + 63
        constexpr int WCP = WST ? C::BN * rb::kWRoundBytes / 1024 : 0;
        const auto wsr = make_rsrc(p.W + (size_t)n0 * col_bytes, (uint32_t)ncols * col_bytes);
        uint32_t wo[WCP ? WCP : 1];
#pragma unroll
        for (int c = 0; c < WCP; c++) {
            const uint32_t u = 64u * c + lane, col = u / 5u, unit = u % 5u;
            wo[c] = col < (uint32_t)ncols ? col * col_bytes + 16u * unit : kOOB;
        }
        auto issue = [&](uint32_t t) {
            if constexpr (WST) {
                if (t % KG == 0) {  // the round's weights ahead of its X
                    const uint32_t q = t / KG;
                    const uint32_t wsoff = (g_begin + 4u * q) * 20u;
                    uint8_t* const wdst = reinterpret_cast<uint8_t*>(lds) + XBYTES + (q % rb::kWStages) * (C::BN * rb::kWRoundBytes);
#pragma unroll
                    for (int c = 0; c < WCP; c++) {
                        const uint32_t vo = wo[c];
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (__attribute__((address_space(3))) void*)(wdst + c * 1024),
                                                                 16, vo, (int)wsoff, 0, 0);
                    }
                }
            }
            const uint32_t soff = (k_begin + t * kBK) * 2u;
            _Float16* const dst = lds + (t % C::XS) * C::LDS_STAGE;
            // a 32-K last step (K % 64 == 32) takes the first-half offsets
            // (K groups take whole 128-K rounds: never, so no per-copy select
            // and its wait state sit between their copies)
            const bool half = KG == 1 && k_begin + t * kBK + kBK > k_end;
#pragma unroll
            for (int q = 0; q < C::XCP; q++) {
                const uint32_t vo = half ? xh[q] : xo[q];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(dst + q * 512),
                                                         16, vo, (int)soff, 0, 0);
            }
        };
        for (uint32_t t = 0; t < (uint32_t)(KG * C::XD) && t < nsteps; t++) issue(t);
        const uint32_t nloc = nsteps / KG;
        for (uint32_t t = 0; t < nloc; t++) {
            // the barrier opening round t needs steps .. KG (t + 2) - 1; copies
            // issued after those: steps KG (t + 2) .. min(KG (t + XD) - 1, nsteps - 1)
            const int r = min(KG * (C::XD - 2), (int)nsteps - KG * ((int)t + 2));
            if constexpr (WST) {  // whole rounds: their weight copies, then their X
                if (r >= KG) rb_wait_vmcnt<KG * C::XCP + WCP>();
                else rb_wait_vmcnt<0>();
            } else {
                if (r >= 3) rb_wait_vmcnt<3 * C::XCP>();
                else if (r == 2) rb_wait_vmcnt<2 * C::XCP>();
                else if (r == 1) rb_wait_vmcnt<C::XCP>();
                else rb_wait_vmcnt<0>();
            }
            asm volatile("s_barrier" ::: "memory");
#pragma unroll
            for (int i = 0; i < KG; i++)
                if (KG * (t + C::XD) + i < nsteps) issue(KG * (t + C::XD) + i);
        }
        return;
    }
    static_assert(!C::XST || (KG * (C::XD - 2) <= 3 && 3 * C::XCP < 64), "stager waits");
    static_assert(!WST || (C::XD - 2 == 1 && KG * C::XCP + C::BN * rb::kWRoundBytes / 1024 < 64), "stager waits (WST)");
    auto wr0 = make_rsrc(p.W + (size_t)n0 * col_bytes, (uint32_t)ncols * col_bytes);
    auto wr1 = make_rsrc(DUAL ? p.W2 + (size_t)n0 * col_bytes : p.W, DUAL ? (uint32_t)ncols * col_bytes : 0u);

    // local column of B tile jb for this lane
    auto bcol = [&](int jb) { return wcolg * C::WN + (jb % TN) * 32 + c32; };

    // Pipelines (U = 6 steps unrolled, so every ring index below is static):
    //  X:  (XST) in LDS stage step % XS, copied there by the stager wave; or
    //      raw 16-byte chunks fetched 4 steps ahead into XP = 2 register slots,
    //      written to LDS 2 steps ahead into a 3-stage ring;
    //  A:  fragments of slice kk + 1 read while slice kk multiplies; the first
    //      slice of step s + 1 is read before the step's barrier (its stage was
    //      written before the previous barrier);
    //  W:  raw blocks fetched WP steps ahead, decoded one step ahead into the
    //      two B buffers.
    constexpr int XS = C::XS, XP = 2, WP = P, U = C::U;
    static_assert((KG * U) % XS == 0 && U % XP == 0 && U % WP == 0, "ring sizes divide the unroll");
    uint32_t xraw[XP][C::XST ? 1 : C::XPT][4];
    uint32_t wraw[WP][NCB][Dec::kRawWords];

    auto load_x = [&](uint32_t step, int slot) {
        if constexpr (!C::XST) {
            const uint32_t k0 = k_begin + step * kBK;
#pragma unroll
            for (int i = 0; i < C::XPT; i++) {
                const int c = tid + NT * i;
                const int row = c >> 3, kc = c & 7;
                const uint32_t k = k0 + kc * 8;  // past the range (or the last step): zeros
                const uint32_t off = ((C::XCH % NT == 0 || c < C::XCH) && k < k_end) ? ((uint32_t)row * K + k) * 2u : kOOB;
                const u4_t v = ld_b128(xr, off);
                xraw[slot][i][0] = v.x; xraw[slot][i][1] = v.y; xraw[slot][i][2] = v.z; xraw[slot][i][3] = v.w;
            }
        }
    };
    // WST: the raw words of this lane's group of local round jr + 1's step
    auto read_w = [&](int jr, int slot) {
        const uint8_t* base = reinterpret_cast<const uint8_t*>(lds) + XBYTES + (jr % rb::kWStages) * (C::BN * rb::kWRoundBytes) +
                              (2 * kg + h) * 20;
#pragma unroll
        for (int jb = 0; jb < NCB; jb++)
#pragma unroll
            for (int i = 0; i < Dec::kRawWords; i++)
                wraw[slot][jb][i] = *reinterpret_cast<const uint32_t*>(base + bcol(jb) * rb::kWRoundBytes + 4 * i);
    };
    auto load_w = [&](uint32_t step, int slot) {
        if constexpr (WST) return;
        const uint32_t g = g_begin + step * 2 + h;
        const bool live = g < g_end;
#pragma unroll
        for (int jb = 0; jb < NCB; jb++) {
            const uint32_t coff = live ? (uint32_t)bcol(jb) * col_bytes : kOOB;
            Dec::load((DUAL && jb >= TN) ? wr1 : wr0, coff, live ? g : 0u, wraw[slot][jb]);
        }
    };

    auto store_x = [&](int slot, int stage) {
        if constexpr (!C::XST) {
            _Float16* As = lds + stage * C::LDS_STAGE;
#pragma unroll
            for (int i = 0; i < C::XPT; i++) {
                const int c = tid + NT * i;
                if (C::XCH % NT == 0 || c < C::XCH) {
                    const int row = c >> 3, kc = c & 7;
                    *reinterpret_cast<u4_t*>(As + row * kLdsRow + kc * 8) =
                        u4_t{xraw[slot][i][0], xraw[slot][i][1], xraw[slot][i][2], xraw[slot][i][3]};
                }
            }
        }
    };

    auto decode = [&](uint32_t step, int slot, uint32_t out[NCB][16]) {
        const uint32_t g = g_begin + step * 2 + h;
#pragma unroll
        for (int jb = 0; jb < NCB; jb++) {
            const uint32_t par = Dec::parity((uint32_t)bcol(jb) * col_bytes, g);
            decode_group<F>(wraw[slot][jb], par, out[jb]);
        }
    };

    f16v_t acc[TM][NCB];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < NCB; j++) acc[i][j] = f16v_t{};

    const int arow = wrow * C::WM + c32;
    const int akof = 32 * h;
    // swizzled stages: the lane's offset (halfs) of row tile i, k-slice kk
    uint32_t aswz[C::XSW ? TM : 1][4];
    if constexpr (C::XSW) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const uint32_t r = (uint32_t)(arow + i * 32);
                aswz[i][kk] = r * kBK + 8u * ((4u * (uint32_t)h + (uint32_t)kk) ^ rb::xswz(r));
            }
    }
    // stage of local round j (static within the unroll) plus the K group
    auto read_a = [&](int j, int kk, h8_t out[TM]) {
        const _Float16* As = lds + ((KG * j) % XS + kg) * C::LDS_STAGE;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if constexpr (C::XSW)
                out[i] = *reinterpret_cast<const h8_t*>(As + aswz[i][kk]);
            else
                out[i] = *reinterpret_cast<const h8_t*>(As + (arow + i * 32) * kLdsRow + akof + kk * 8);
        }
    };

    uint32_t bw[2][NCB][16];
    h8_t af[2][TM];

    // One K step, as four k-slices.  Slice kk: read the A fragments of slice
    // kk + 1 (of step s + 1 for the last slice), the TM x NCB MFMAs of slice kk,
    // one half-group decode of step s + 1 and a share of the memory traffic
    // (W fetch of step s + 1 + WP, X store of step s + 2, X fetch of step s + 4).
    // Each slice is a fenced scheduling region in which MFMAs and decode VALU
    // ops alternate, so the decode issues while the matrix pipe is busy.
    constexpr int NM = TM * NCB;            // MFMAs per slice
    constexpr int HALVES = 2 * NCB;         // half-group decodes per step
    constexpr int DPS = (HALVES + 3) / 4;   // half-group decodes per slice
    auto step_body = [&](uint32_t s, int j) {
        const int wslot = (j + 1) % WP;
        if constexpr (WST) read_w(j + 1, wslot);  // the next round's weights (visible since this round's barrier)
        uint32_t (*bn)[16] = bw[(j + 1) & 1];
        const uint32_t gn = g_begin + (s + KG) * 2 + h;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            __builtin_amdgcn_sched_barrier(0);
            if (kk < 3) read_a(j, kk + 1, af[(kk + 1) & 1]);
            else read_a(j + 1, 0, af[0]);
#pragma unroll
            for (int jb = 0; jb < NCB; jb++) {
                const uint32_t* bj = bw[j & 1][jb];
                const h8_t b = __builtin_bit_cast(h8_t, u4_t{bj[4 * kk], bj[4 * kk + 1], bj[4 * kk + 2], bj[4 * kk + 3]});
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[i][jb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk & 1][i], b, acc[i][jb], 0, 0, 0);
            }
#pragma unroll
            for (int d = kk * DPS; d < (kk + 1) * DPS && d < HALVES; d++) {
                const int jb = d >> 1, hh = d & 1;
                const uint32_t par = Dec::parity((uint32_t)bcol(jb) * col_bytes, gn);
                decode_half_fast<F>(wraw[wslot][jb], par, hh, bn[jb] + 8 * hh);
            }
            if (kk == 1) store_x((j + 2) % XP, (j + 2) % XS);
            if (kk == 2) load_x(s + 2 + XP, (j + 2) % XP);
            __builtin_amdgcn_sched_group_barrier(0x100, TM, 0);  // DS read
#pragma unroll
            for (int q = 0; q < NM; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, KG > 1 ? kVpmKG : kVpm, 0);  // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (F == QUANT_Q4_K || F == QUANT_Q4_0) {
            // wave-uniform slow path: re-decode exactly when any lane's group
            // needs it (Q4_K binade gap; Q4_0 scales with -8 d not finite).
            // The exact words replace the fast ones per lane through a select,
            // so the fast words stay live on both paths: overwritten outright,
            // the compiler sinks the fast decode into the not-slow branch,
            // behind the step's MFMAs, where it no longer issues under them.
            bool slow[NCB], any_slow = false;
#pragma unroll
            for (int jb = 0; jb < NCB; jb++) {
                slow[jb] = needs_exact<F>(wraw[wslot][jb], Dec::parity((uint32_t)bcol(jb) * col_bytes, gn));
                any_slow |= slow[jb];
            }
            if (__any(any_slow)) {
#pragma unroll
                for (int jb = 0; jb < NCB; jb++) {
                    uint32_t ex[16];
                    decode_group<F>(wraw[wslot][jb], Dec::parity((uint32_t)bcol(jb) * col_bytes, gn), ex);
#pragma unroll
                    for (int w = 0; w < 16; w++) bn[jb][w] = slow[jb] ? ex[w] : bn[jb][w];
                }
            }
        }
        load_w(s + KG * (1 + WP), wslot);
        __syncthreads();
    };

    // ---- prologue ----
#pragma unroll
    for (int t = 0; t < XP; t++) load_x(t, t);
#pragma unroll
    for (int t = 0; t < WP; t++) load_w(KG * t + kg, t);
    store_x(0, 0);
    store_x(1, 1);
    load_x(XP, 0);
    load_x(XP + 1, 1);
    if constexpr (WST) {
        __syncthreads();
        read_w(0, 0);
        decode(kg, 0, bw[0]);
    } else {
        decode(kg, 0, bw[0]);
        load_w(KG * WP + kg, 0);
        __syncthreads();
    }
    read_a(0, 0, af[0]);

    // ---- main loop: full groups of U steps branch-free (look-ahead fetches past
    // the K range read zeros), then the remainder with guards ----
    // rounds of KG steps: this wave takes step KG t + kg of round t
    const uint32_t nloc = nsteps / KG;
    uint32_t t0 = 0;
    for (; t0 + U <= nloc; t0 += U) {
#pragma unroll
        for (int j = 0; j < U; j++) step_body(KG * (t0 + j) + kg, j);
    }
#pragma unroll
    for (int j = 0; j < U; j++)
        if (t0 + j < nloc) step_body(KG * (t0 + j) + kg, j);

    // ---- K groups: group 1 hands its tile to group 0 through LDS (every
    // wave is past the last step's barrier, so the X stages are free) ----
    if constexpr (KG > 1) {
        static_assert(KG == 2, "two K groups");
        float* const xg = reinterpret_cast<float*>(lds) + wl * (C::ACC * 64);
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < NCB; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *reinterpret_cast<f4_t*>(xg + (((i * NCB + j) * 4 + q) * 64 + lane) * 4) =
                            f4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
        __syncthreads();
        if (kg == 1) return;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < NCB; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f4_t o = *reinterpret_cast<const f4_t*>(xg + (((i * NCB + j) * 4 + q) * 64 + lane) * 4);
                    acc[i][j][4 * q] += o.x;
                    acc[i][j][4 * q + 1] += o.y;
                    acc[i][j][4 * q + 2] += o.z;
                    acc[i][j][4 * q + 3] += o.w;
                }
    }

    // ---- split-K: this split's fp32 partial sums go to the workspace, laid
    // out [split][plane][M][N] (plane 1: the SwiGLU up projection); the
    // reduction kernel launched after this one (splitk_reduce_kernel) sums
    // the splits in split order and runs the epilogue.  The kernel boundary
    // orders the partials before their reads: no cross-workgroup
    // synchronization inside the kernel.  Lanes 0..31 of a row store 128
    // consecutive bytes. ----
    if (SPLIT && ksplit > 1) {
        const size_t plane = (size_t)M * N;
        float* base = p.ws + (size_t)kz * plane * (DUAL ? 2 : 1);
        const int r0 = m0 + wrow * C::WM, c0 = n0 + wcolg * C::WN;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int jb = 0; jb < NCB; jb++) {
                const int n = c0 + (jb % TN) * 32 + c32;
                float* pl = base + (DUAL && jb >= TN ? plane : 0);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = r0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < (int)M && n < (int)N) pl[(size_t)m * N + n] = acc[i][jb][r];
                }
            }
        return;
    }

    // ---- epilogue: accumulator element r of lane l is row 8 (r / 4) + 4 (l / 32)
    // + r % 4, column l % 32 of its 32x32 tile.  Values (SwiGLU-combined) go
    // through LDS one 32-row band of the wave tile at a time, so each lane then
    // owns 8 consecutive columns of one row: residual read and output written
    // with 16-byte accesses, one rounding to fp16 after the residual add. ----
    auto value = [&](int i, int j, int r) {
        float v = acc[i][j][r];
        if constexpr (DUAL) {
            const float u = acc[i][j + TN][r];
            v = silu_mul(v, u);
        }
        return v;
    };
    const int wcol0 = n0 + wcolg * C::WN;
    const int wrow0 = m0 + wrow * C::WM;
    const bool vec_io = ((reinterpret_cast<uintptr_t>(p.Y) | reinterpret_cast<uintptr_t>(p.R)) & 15u) == 0 &&
                        (N & 7u) == 0 && (p.head_D & 7u) == 0;
    if (vec_io) {
        constexpr int WC = C::WN;
        constexpr int ERS = C::ERS, EJS = C::EJS;
        static_assert(NW * 32 * ERS * 4 <= C::LDS_BYTES, "epilogue staging fits the LDS allocation");
        float* E = reinterpret_cast<float*>(lds) + wave * 32 * ERS;
        __syncthreads();  // every wave is done with the X stages
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    E[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * ERS + j * EJS + c32] = value(i, j, r);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS writes done (wave-local region)
            __builtin_amdgcn_wave_barrier();
            constexpr int CHUNKS = 32 * WC / 8;
#pragma unroll
            for (int c = lane; c < CHUNKS; c += 64) {
                const int row = c / (WC / 8), c8 = c % (WC / 8);
                const int m = wrow0 + i * 32 + row;
                const int n = wcol0 + c8 * 8;
                if (m < (int)M && n < (int)N) {
                    // Half of the lanes of a read pass take their upper four
                    // columns first (odd rows with one tile per wave, odd
                    // tiles otherwise), so one pass covers every bank.
                    const float* e = E + row * ERS + (c8 >> 2) * EJS + (c8 & 3) * 8;
                    const int sw = (TN == 1 ? row : (c8 >> 2)) & 1;
                    const f4_t a = *reinterpret_cast<const f4_t*>(e + 4 * sw);
                    const f4_t b = *reinterpret_cast<const f4_t*>(e + 4 - 4 * sw);
                    const f4_t lo = sw ? b : a, hi = sw ? a : b;
                    float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    if (p.R) {
                        const u4_t rr = *reinterpret_cast<const u4_t*>(p.R + (size_t)m * N + n);
                        const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const h2_t hh = as_h2(rw[q]);
                            v[2 * q] += (float)hh.x;
                            v[2 * q + 1] += (float)hh.y;
                        }
                    }
                    u4_t o;
                    o.x = pack_h2(f2h_bits(v[0]), f2h_bits(v[1]));
                    o.y = pack_h2(f2h_bits(v[2]), f2h_bits(v[3]));
                    o.z = pack_h2(f2h_bits(v[4]), f2h_bits(v[5]));
                    o.w = pack_h2(f2h_bits(v[6]), f2h_bits(v[7]));
                    size_t off;
                    if (p.head_D) {
                        const uint32_t hd = (uint32_t)n / p.head_D, dd = (uint32_t)n % p.head_D;
                        off = ((size_t)hd * M + m) * p.head_D + dd;
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
            const int n = wcol0 + j * 32 + c32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = wrow0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < (int)M && n < (int)N) {
                    float v = value(i, j, r);
                    if (p.R) v += (float)p.R[(size_t)m * N + n];
                    size_t o;
                    if (p.head_D) {
                        const uint32_t hd = (uint32_t)n / p.head_D, dd = (uint32_t)n % p.head_D;
                        o = ((size_t)hd * M + m) * p.head_D + dd;
                    } else {
                        o = (size_t)m * N + n;
                    }
                    p.Y[o] = (_Float16)v;
                }
            }
        }
}


template <int F, int TM, int TN, int NW, int WR, int KG, bool DUAL>
static hipError_t rb_launch_cfg(const GemmParams& p, hipStream_t st) {
    using C = rb::Cfg<TM, TN, NW, WR, KG, DUAL, rb::use_stager(F, TN, NW, KG, DUAL)>;
    auto kern = gemm_rb_kernel<F, TM, TN, NW, WR, KG, DUAL, kWeightStages, false>;
    if constexpr (KG > 1) {
        if (p.ksplit > 1 || p.K % (64 * KG) != 0) return hipErrorInvalidValue;  // rb_pick never asks for these
    } else {
        if (p.ksplit > 1) kern = gemm_rb_kernel<F, TM, TN, NW, WR, KG, DUAL, kWeightStages, true>;
    }
    constexpr bool WST = rb::use_wstage(F, KG, C::XST);
    constexpr size_t LX = (size_t)C::XS * C::LDS_STAGE * 2 + (WST ? rb::kWStages * C::BN * rb::kWRoundBytes : 0);
    const size_t lds = LX > (size_t)C::LDS_BYTES ? LX : (size_t)C::LDS_BYTES;
    const uint32_t ntm = (p.M + C::BM - 1) / C::BM;
    uint32_t T = ntm * ((p.N + C::BN - 1) / C::BN);
    for (uint32_t g = 1; g < p.ngroups && g < 3; g++) T += ntm * ((p.Nx[g - 1] + C::BN - 1) / C::BN);
    const uint32_t ks = p.ksplit ? p.ksplit : 1;
    static size_t attr[2][kMaxDevices] = {};
    const hipError_t e = lds_limit_once((const void*)kern, lds, attr[p.ksplit > 1]);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(T, ks), dim3(C::NTL), lds, st, p);
    return hipGetLastError();
}

template <int F, bool DUAL>
static hipError_t rb_launch_fmt(const GemmParams& p, hipStream_t st) {
    if constexpr (DUAL) {
        return rb_launch_cfg<F, QR_RB_DUAL, true>(p, st);
    } else if constexpr (F == QUANT_VAR_RATE_AFFINE || F == QUANT_EXL3) {
        return rb_launch_cfg<F, QR_RB_MID, false>(p, st);  // rb_pick's only shape for these formats
    } else {
        switch (rb_pick(F, p.M, p.N, p.K, false)) {
            case 0: return rb_launch_cfg<F, QR_RB_BIG, false>(p, st);
            case 3: return rb_launch_cfg<F, QR_RB_BIG_K, false>(p, st);
            case 4: return rb_launch_cfg<F, QR_RB_MID64, false>(p, st);
            case 5: return rb_launch_cfg<F, QR_RB_KG, false>(p, st);
            case 6: return rb_launch_cfg<F, QR_RB_MID64_KG, false>(p, st);
            default: return rb_launch_cfg<F, QR_RB_MID, false>(p, st);
        }
    }
}

template <int F>
hipError_t launch_gemm_format(const GemmParams& p, hipStream_t st) {
    return p.W2 ? rb_launch_fmt<F, true>(p, st) : rb_launch_fmt<F, false>(p, st);
}

#ifndef QR_GEMM_FORMAT
#error "build qr_gemm.hip with -DQR_GEMM_FORMAT=<format id>"
#endif
template hipError_t launch_gemm_format<QR_GEMM_FORMAT>(const GemmParams& p, hipStream_t st);

}  // namespace qr
