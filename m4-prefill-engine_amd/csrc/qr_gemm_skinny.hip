// qr_gemm_skinny.hip -- weight-streaming projection for small M (M <= 64).
//
// The M=33 prefill projection is bound by streaming the
// packed weights from HBM; the reference's 64x64 tiling (quant_router_kernels.
// metal:442-581) leaves 31 of 64 rows idle and launches only N/64 groups.
// Here every CU streams its own slice of W:
//  * a workgroup = 8 wave64s owns 64 output columns and a K range of KC
//    elements; the K range is split across KSPLIT workgroups so the grid
//    covers the 256 CUs;
//  * load phase: the workgroup's 64 weight strips (one contiguous byte range
//    per column) and its activation rows (M x KC fp16) are copied to LDS with
//    fully coalesced 16-byte buffer loads -- every wave keeps its whole share
//    in flight at once; strips and rows are padded by 16 bytes so the
//    fragment reads below spread over the LDS banks;
//  * compute phase: wave w takes groups [w*GPW, (w+1)*GPW) of the range.
//    Weights are the A operand of v_mfma_f32_16x16x32_f16 (16 columns x one
//    32-element quant group): each lane reads the raw bytes of its 8 elements
//    from LDS and decodes them to binary16 in registers (bit-exact vs the CPU
//    unpack); activations are the B operand, 16 rows per tile, reused across
//    the wave's 4 column tiles;
//  * partial sums: the 8 waves reduce through LDS in a fixed order; with a K
//    split, each workgroup writes its fp32 partials to a workspace and the
//    split-K reduction kernel (qr_gemm_host.hip) sums the splits in split
//    order and rounds once to fp16 -- deterministic.
#include "qr_device.h"
#include "qr_formats.h"
#include "qr_kernels.h"

namespace qr {

__device__ __forceinline__ uint32_t lds32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// A-operand fragment of one 32-element group, read from a weight strip in LDS
// (16-byte aligned).  Lane group g = lane / 16 holds elements 8g .. 8g+7, so
// the lane's activations are one 16-byte run.  In the 4-bit formats those are
// nibble g / 2 of code bytes 8 (g & 1) .. 8 (g & 1) + 7 (code byte j holds
// elements j and 16 + j).
// load() reads the raw words of one lane from LDS; decode() is lane-local.
template <int F> struct Frag;

// Q4_0 (18-byte groups, 2-byte aligned): the lane's two code dwords sit at a
// wave-uniform byte shift from the three aligned dwords read; a fourth read
// fetches the dword holding the scale.
template <> struct Frag<QUANT_Q4_0> {
    static constexpr int kRaw = 4;
    __device__ static void load(const uint8_t* strip, uint32_t kb, int g, uint32_t raw[4]) {
        const uint8_t* p = strip + ((kb * 18u + 2u + 8u * ((uint32_t)g & 1u)) & ~3u);
        raw[0] = lds32(p); raw[1] = lds32(p + 4); raw[2] = lds32(p + 8);
        raw[3] = lds32(strip + ((kb * 18u) & ~3u));  // dword holding the scale
    }
    __device__ static h8_t decode(const uint32_t raw[4], uint32_t kb, int g) {
        const uint32_t sh = (kb * 18u + 2u) & 2u, ns = 4u * ((uint32_t)g >> 1);
        const uint32_t lo = (__builtin_amdgcn_alignbyte(raw[1], raw[0], sh) >> ns) & 0x0f0f0f0fu;
        const uint32_t hi = (__builtin_amdgcn_alignbyte(raw[2], raw[1], sh) >> ns) & 0x0f0f0f0fu;
        const uint32_t d16 = ((kb * 18u) & 2u) ? (raw[3] >> 16) : (raw[3] & 0xffffu);
        const h2_t d = as_h2(d16 | (d16 << 16));
        u4_t o;
        if (__all(__builtin_fabsf(h2f(d16)) <= kQ4_0FastMaxScale)) {  // fma(q, d, -8d): -8d exact
            const h2_t m8 = {(_Float16)-8.0f, (_Float16)-8.0f};
            const h2_t c = d * m8;
            o = u4_t{as_u32(__builtin_elementwise_fma(code_pair<false>(lo), d, c)),
                     as_u32(__builtin_elementwise_fma(code_pair<true>(lo), d, c)),
                     as_u32(__builtin_elementwise_fma(code_pair<false>(hi), d, c)),
                     as_u32(__builtin_elementwise_fma(code_pair<true>(hi), d, c))};
        } else {  // (q - 8) * d
            const h2_t off = {(_Float16)8.0f, (_Float16)8.0f};
            o = u4_t{as_u32((code_pair<false>(lo) - off) * d), as_u32((code_pair<true>(lo) - off) * d),
                     as_u32((code_pair<false>(hi) - off) * d), as_u32((code_pair<true>(hi) - off) * d)};
        }
        return __builtin_bit_cast(h8_t, o);
    }
};

// MLX_4BIT (20-byte groups, dword aligned): every lane reads {d, bias} and
// its two code dwords.
template <> struct Frag<QUANT_MLX_4BIT> {
    static constexpr int kRaw = 3;
    __device__ static void load(const uint8_t* strip, uint32_t kb, int g, uint32_t raw[3]) {
        const uint8_t* p = strip + kb * 20u;
        raw[0] = lds32(p);
        raw[1] = lds32(p + 4u + 8u * ((uint32_t)g & 1u));
        raw[2] = lds32(p + 8u + 8u * ((uint32_t)g & 1u));
    }
    __device__ static h8_t decode(const uint32_t raw[3], uint32_t, int g) {
        const uint32_t db = raw[0], ns = 4u * ((uint32_t)g >> 1);
        const uint32_t lo = (raw[1] >> ns) & 0x0f0f0f0fu, hi = (raw[2] >> ns) & 0x0f0f0f0fu;
        const uint32_t d16 = db & 0xffffu, b16 = db >> 16;
        const h2_t d = as_h2(d16 | (d16 << 16)), bias = as_h2(b16 | (b16 << 16));
        u4_t w = {as_u32(__builtin_elementwise_fma(code_pair<false>(lo), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<true>(lo), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<false>(hi), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<true>(hi), d, bias))};
        return __builtin_bit_cast(h8_t, w);
    }
};

// Q4_K: group kb is sub-block s = kb % 8 of super-block kb / 8.  Every lane
// reads the 16-byte header and its two code dwords of the sub-block (bytes
// 16 + 16s + 8 (g & 1) .. +7).
template <> struct Frag<QUANT_Q4_K> {
    static constexpr int kRaw = 6;
    __device__ static void load(const uint8_t* strip, uint32_t kb, int g, uint32_t raw[6]) {
        const uint8_t* p = strip + (kb >> 3) * 144u;
        u4_t h = *reinterpret_cast<const u4_t*>(p);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = lds32(p + 16u + 16u * (kb & 7u) + 8u * ((uint32_t)g & 1u));
        raw[5] = lds32(p + 20u + 16u * (kb & 7u) + 8u * ((uint32_t)g & 1u));
    }
    __device__ static int binade(uint32_t h16) {
        int e = (int)((h16 >> 10) & 0x1f);
        return (e < 1 ? 1 : e) - 15;
    }
    __device__ static h8_t decode(const uint32_t raw[6], uint32_t kb, int g) {
        const uint32_t s = kb & 7u;
        const uint32_t d16 = raw[0] & 0xffffu, dm16 = raw[0] >> 16;
        const uint64_t s07 = (uint64_t)raw[1] | ((uint64_t)raw[2] << 32);
        const uint32_t scj = (uint32_t)(s07 >> (8u * s)) & 0xffu;
        const uint32_t sc = scj & 63u;
        const uint32_t lowm = (s < 4) ? ((raw[3] >> (8u * s)) & 0x0fu) : ((raw[3] >> (8u * (s - 4u) + 4u)) & 0x0fu);
        const uint32_t mn = lowm | ((scj >> 6) << 4);
        const float A = h2f(d16) * (float)sc;
        const float B = h2f(dm16) * (float)mn;
        const int gap = binade(d16) - binade(dm16);
        const bool fast = (A == 0.0f) || (B == 0.0f) || (gap <= 3 && gap >= -7);
        const uint32_t ns = 4u * ((uint32_t)g >> 1);
        const uint32_t q0 = (raw[4] >> ns) & 0x0f0f0f0fu, q1 = (raw[5] >> ns) & 0x0f0f0f0fu;
        u4_t w;
        if (__all(fast)) {  // exact-sum path only when some lane needs it
            w = u4_t{affine_pair_exact(code_pair<false>(q0), A, -B), affine_pair_exact(code_pair<true>(q0), A, -B),
                     affine_pair_exact(code_pair<false>(q1), A, -B), affine_pair_exact(code_pair<true>(q1), A, -B)};
        } else {
            w = u4_t{affine_pair_any(code_pair<false>(q0), A, -B, fast), affine_pair_any(code_pair<true>(q0), A, -B, fast),
                     affine_pair_any(code_pair<false>(q1), A, -B, fast), affine_pair_any(code_pair<true>(q1), A, -B, fast)};
        }
        return __builtin_bit_cast(h8_t, w);
    }
};

// TERNARY_1_58 (12-byte groups): elements 8g..8g+7 are the 16-bit field
// 16(g&1) of code word g/2.  w = (1024 + c - 1025) * d, exact.
template <> struct Frag<QUANT_TERNARY_1_58> {
    static constexpr int kRaw = 2;
    __device__ static void load(const uint8_t* strip, uint32_t kb, int g, uint32_t raw[2]) {
        const uint8_t* p = strip + kb * 12u;
        raw[0] = lds32(p);
        raw[1] = lds32(p + 4u + 4u * (uint32_t)(g >> 1));
    }
    __device__ static h8_t decode(const uint32_t raw[2], uint32_t, int g) {
        const uint32_t d16 = raw[0] & 0xffffu;
        const uint32_t c = (raw[1] >> (16 * (g & 1))) & 0xffffu;
        const h2_t d = as_h2(d16 | (d16 << 16));
        const h2_t off = {(_Float16)1025.0f, (_Float16)1025.0f};
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t t = (c >> (4 * i)) & 0xfu;
            const uint32_t pr = (t & 3u) | ((t >> 2) << 16) | 0x64006400u;
            w[i] = as_u32((as_h2(pr) - off) * d);
        }
        return __builtin_bit_cast(h8_t, u4_t{w[0], w[1], w[2], w[3]});
    }
};


// MLX_4BIT_G64 (36-byte 64-element blocks): group kb is half kb % 2 of block
// kb / 2; lane group g takes code word 4 (kb % 2) + g, i.e. elements
// 8g .. 8g + 7 of the group, in element order (two byte permutes).
template <> struct Frag<QUANT_MLX_4BIT_G64> {
    static constexpr int kRaw = 2;
    __device__ static void load(const uint8_t* strip, uint32_t kb, int g, uint32_t raw[2]) {
        const uint8_t* p = strip + (kb >> 1) * 36u;
        raw[0] = lds32(p);
        raw[1] = lds32(p + 4u + 16u * (kb & 1u) + 4u * (uint32_t)g);
    }
    __device__ static h8_t decode(const uint32_t raw[2], uint32_t, int) {
        const uint32_t d16 = raw[0] & 0xffffu, b16 = raw[0] >> 16;
        const h2_t d = as_h2(d16 | (d16 << 16)), bias = as_h2(b16 | (b16 << 16));
        const uint32_t lo = raw[1] & 0x0f0f0f0fu, hi = (raw[1] >> 4) & 0x0f0f0f0fu;
        const uint32_t a = perm(hi, lo, 0x05010400u), b = perm(hi, lo, 0x07030602u);
        u4_t w = {as_u32(__builtin_elementwise_fma(code_pair<false>(a), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<true>(a), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<false>(b), d, bias)),
                  as_u32(__builtin_elementwise_fma(code_pair<true>(b), d, bias))};
        return __builtin_bit_cast(h8_t, w);
    }
};

constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkNT = 4;                  // 16-column tiles per wave
constexpr int kSkCols = 16 * kSkNT;       // columns per workgroup
constexpr uint32_t kSkLdsMax = 159 * 1024;  // 160 KB LDS less static allocations

// Bytes of one 32-element group of format F.
template <int F> struct GroupBytes;
template <> struct GroupBytes<QUANT_Q4_0> { static constexpr uint32_t v = 18; };
template <> struct GroupBytes<QUANT_MLX_4BIT> { static constexpr uint32_t v = 20; };
template <> struct GroupBytes<QUANT_Q4_K> { static constexpr uint32_t v = 18; };  // 144 / 8
template <> struct GroupBytes<QUANT_TERNARY_1_58> { static constexpr uint32_t v = 12; };
template <> struct GroupBytes<QUANT_MLX_4BIT_G64> { static constexpr uint32_t v = 18; };  // 36 / 2

// LDS layout of one launch: activation rows [M][KC*2 + 16 bytes], then 64
// weight strips [64][SB + 16 bytes]; the wave reduction reuses it from 0.
struct SkLayout {
    uint32_t xrs, sb, sbp, x_bytes, lds;
};
__host__ __device__ inline SkLayout sk_layout(uint32_t M, uint32_t gpw, uint32_t group_bytes) {
    SkLayout L;
    const uint32_t kc = gpw * kSkWaves * 32;
    L.xrs = kc * 2 + 16;
    L.sb = gpw * kSkWaves * group_bytes;
    L.sbp = L.sb + 16;
    L.x_bytes = M * L.xrs;
    const uint32_t mt = (M + 15) / 16;
    const uint32_t red = kSkWaves * mt * 16 * (kSkCols + 4) * 4;
    const uint32_t load = L.x_bytes + kSkCols * L.sbp;
    L.lds = load > red ? load : red;
    return L;
}

template <int F, int MT, int GPW>  // MT: 16-row tiles of M; GPW: 32-groups per wave
__global__ void __launch_bounds__(kSkThreads) gemm_skinny_kernel(GemmParams p, float* ws, uint32_t ksplit) {
    using FR = Frag<F>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr uint32_t GB = GroupBytes<F>::v;
    constexpr uint32_t KC = GPW * kSkWaves * 32;      // K elements of this workgroup
    constexpr uint32_t SB = GPW * kSkWaves * GB;      // strip bytes (multiple of 16)
    static_assert(SB % 16 == 0, "strip bytes must be a multiple of 16");

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t cg = blockIdx.x, ks = blockIdx.y;
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t n0 = cg * kSkCols;
    const uint32_t col_bytes = (uint32_t)p.col_bytes;
    const uint32_t ncols = min((uint32_t)kSkCols, N - n0);
    const SkLayout L = sk_layout(M, GPW, GB);
    uint8_t* xs = smem;
    uint8_t* wsb = smem + L.x_bytes;

    // ---- load phase: strips and rows to LDS, all loads in flight ----
    {
        auto wr = make_rsrc(p.W + (size_t)n0 * col_bytes, ncols * col_bytes);
        auto xr = make_rsrc(p.X, M * K * 2u);
        constexpr uint32_t WCH = kSkCols * SB / 16;       // 16-byte chunks of the strips
        constexpr uint32_t WPT = (WCH + kSkThreads - 1) / kSkThreads;
        constexpr uint32_t xch_row = KC * 2 / 16;
        const uint32_t XCH = M * xch_row;
        constexpr uint32_t XPT_MAX = (MT * 16 * xch_row + kSkThreads - 1) / kSkThreads;
        u4_t wv[WPT], xv[XPT_MAX];
#pragma unroll
        for (uint32_t i = 0; i < WPT; i++) {
            const uint32_t q = tid + kSkThreads * i;
            const uint32_t c = q / (SB / 16), j = q % (SB / 16);
            const uint32_t off = (q < WCH && c < ncols) ? c * col_bytes + ks * SB + 16 * j : kOOB;
            wv[i] = ld_b128(wr, off);
        }
#pragma unroll
        for (uint32_t i = 0; i < XPT_MAX; i++) {
            const uint32_t q = tid + kSkThreads * i;
            const uint32_t m = q / xch_row, j = q % xch_row;
            const uint32_t off = (q < XCH) ? (m * K + ks * KC) * 2u + 16 * j : kOOB;
            xv[i] = ld_b128(xr, off);
        }
#pragma unroll
        for (uint32_t i = 0; i < WPT; i++) {
            const uint32_t q = tid + kSkThreads * i;
            if (q < WCH) *reinterpret_cast<u4_t*>(wsb + (q / (SB / 16)) * L.sbp + 16 * (q % (SB / 16))) = wv[i];
        }
#pragma unroll
        for (uint32_t i = 0; i < XPT_MAX; i++) {
            const uint32_t q = tid + kSkThreads * i;
            if (q < XCH) *reinterpret_cast<u4_t*>(xs + (q / xch_row) * L.xrs + 16 * (q % xch_row)) = xv[i];
        }
    }
    __syncthreads();

    // ---- compute phase: acc[t][mt] rows n = 16t + 4g + i, column m = 16mt + r16 ----
    f4_t acc[kSkNT][MT];
#pragma unroll
    for (int t = 0; t < kSkNT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[t][mt] = f4_t{};
    // All LDS reads of the wave first (one latency), then decode + MFMA.
    uint32_t raw[GPW][kSkNT][FR::kRaw];
    u4_t xf[GPW][MT];
#pragma unroll
    for (int b = 0; b < GPW; b++) {
        const uint32_t kb = wave * GPW + b;  // group within the workgroup's range
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t m = min(16u * mt + r16, M - 1);  // rows >= M are zeroed below
            xf[b][mt] = *reinterpret_cast<const u4_t*>(xs + m * L.xrs + (kb * 32u + 8u * g) * 2u);  // k = 8g .. 8g + 7
        }
#pragma unroll
        for (int t = 0; t < kSkNT; t++) FR::load(wsb + (16u * t + r16) * L.sbp, kb, g, raw[b][t]);
    }
#pragma unroll
    for (int b = 0; b < GPW; b++) {
        const uint32_t kb = wave * GPW + b;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            if (16u * mt + r16 >= M) xf[b][mt] = u4_t{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < kSkNT; t++) {
            const h8_t a = FR::decode(raw[b][t], kb, g);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8_t, xf[b][mt]),
                                                                   acc[t][mt], 0, 0, 0);
        }
    }

    // ---- reduce the 8 waves through LDS (fixed order) ----
    // Per-wave buffer [m][n] with row stride RS = 64 + 4 floats: a lane's four
    // accumulator rows are 4 consecutive n, stored with one ds_write_b128; the
    // summing pass reads consecutive n (conflict-free) and the outputs leave
    // in row-major order.
    constexpr int ROWS = MT * 16;
    constexpr int RS = kSkCols + 4;
    float* red = reinterpret_cast<float*>(smem);
    __syncthreads();  // every wave is done reading the staged operands
    float* mine = red + wave * ROWS * RS;
#pragma unroll
    for (int t = 0; t < kSkNT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            *reinterpret_cast<f4_t*>(mine + (16 * mt + r16) * RS + 16 * t + 4 * g) = acc[t][mt];
    __syncthreads();

    const bool split = ksplit > 1;
    constexpr int NEL = ROWS * kSkCols;
    constexpr int PER = (NEL + kSkThreads - 1) / kSkThreads;  // outputs per thread; element idx -> (m = idx / 64, n = idx % 64)
    // K split: this split's fp32 partials go to ws [split][M][N] and
    // splitk_reduce_kernel (launched next) sums them in split order;
    // otherwise the sum is the output.
    float* part = split ? ws + (size_t)ks * M * N : nullptr;
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int idx = tid + kSkThreads * e;
        const uint32_t m = idx / kSkCols, nl = idx % kSkCols;
        if (idx >= NEL || m >= M || nl >= ncols) continue;
        const int off = (idx / kSkCols) * RS + idx % kSkCols;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kSkWaves; w++) v += red[w * ROWS * RS + off];
        const uint32_t n = n0 + nl;
        if (split) {
            part[(size_t)m * N + n] = v;
            continue;
        }
        if (p.R) v += (float)p.R[(size_t)m * N + n];
        size_t o;
        if (p.head_D) {
            const uint32_t h = n / p.head_D, dd = n % p.head_D;
            o = ((size_t)h * M + m) * p.head_D + dd;
        } else {
            o = (size_t)m * N + n;
        }
        p.Y[o] = (_Float16)v;
    }
}

// ---- single-kernel streaming projection (no K split) ----
// A workgroup of 8 wave64s owns 16 output columns over the whole of K, so no
// two workgroups share an output and no second kernel sums partials:
//  * the 16 columns' weights are one contiguous byte run of W; it is copied
//    to LDS first, in address order (padded by 16 bytes per column), by
//    buffer-load-to-LDS (16 bytes per lane, no register round trip);
//  * K then advances in NCH chunks of 256 (8 quant groups): each chunk's
//    activation rows (512 bytes each, two rows per 64-lane copy, the 16-byte
//    units of row r XOR-swizzled by r mod 16 so the fragment reads of 16 rows
//    hit distinct banks; rows past M are copied as zeros and their lanes read
//    no fragment) go to a ring of S slots, S - 1 chunks in flight;
//  * one barrier per chunk orders every wave's copies of chunk c before the
//    reads and every wave's reads of chunk c - 1 before the copy of chunk
//    c + S - 1 into that slot; each wave waits for its own copies with an
//    immediate vmcnt (copies retire in order);
//  * every lane's copy offsets and LDS read offsets are formed once; a copy is
//    one instruction with the chunk's K offset in the scalar soffset field,
//    and every trip count is a compile-time constant (copy loops with runtime
//    trip counts issued at about half the rate);
//  * wave w decodes group w of the chunk (A operand, Frag<F>) once and
//    multiplies it with every row tile (B operand): each weight is decoded
//    once per workgroup (two waves per group doubled the decode VALU per
//    SIMD, which bounds this loop);
//  * the workgroups of one XCD (blockIdx % 8) start at successive chunks (the
//    K order is rotated), so the CUs sharing an L2 stream different lines of X;
//  * the 8 group partials of every output meet in LDS in a fixed order.
// Each CU reads all of X (M K 2 bytes, from L2) beside its 16 K GB / 32 bytes
// of W: the trade that removes the split-K partials and their kernel.
constexpr int kStWaves = 8;  // one per quant group of a chunk
constexpr int kStThreads = 64 * kStWaves;
constexpr int kStCols = 16;
constexpr uint32_t kStKC = 256;               // K per chunk
constexpr uint32_t kStLdsMax = 160 * 1024;

template <int F, int MT, int NCH>
struct StShape {
    static constexpr uint32_t GB = GroupBytes<F>::v;
    static constexpr uint32_t CB = NCH * 8 * GB;                    // column bytes
    static constexpr uint32_t WROW = CB + 16;                       // padded column in LDS
    static constexpr uint32_t WI = (kStCols * WROW / 16 + 63) / 64; // 64-lane copies of W
    static constexpr uint32_t WPW = (WI + kStWaves - 1) / kStWaves;
    static constexpr uint32_t WBYTES = WI * 1024;
    static constexpr uint32_t XI = 8 * MT;                          // copies per chunk (two rows each)
    static constexpr uint32_t XPW = (XI + kStWaves - 1) / kStWaves;  // copy rounds per chunk
    static constexpr uint32_t SLOT = XI * 1024;
    static constexpr uint32_t S0 = WBYTES < kStLdsMax ? (kStLdsMax - WBYTES) / SLOT : 0;
    static constexpr uint32_t S = S0 > 8 ? 8 : S0;                  // ring depth
    static constexpr uint32_t RED = 8 * MT * 16 * (kStCols + 4) * 4;
    static constexpr uint32_t LDS = (WBYTES + S * SLOT) > RED ? WBYTES + S * SLOT : RED;
};

// s_waitcnt vmcnt(N), N an immediate.
template <uint32_t N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that is also a compiler barrier for memory accesses (LDS
// reads after it stay after it; copies into a freed slot stay after it).
__device__ __forceinline__ void barrier_mem() { asm volatile("s_barrier" ::: "memory"); }

template <int F, int MT, int NCH>
__global__ void __launch_bounds__(kStThreads, 1) gemm_stream_kernel(GemmParams p) {
    using FR = Frag<F>;
    // The shape's constants as local constexprs: naming a class template's
    // static members in kernel code made the host pass drop the kernel stub
    // silently (the library then linked with the kernel undefined).
    using SH = StShape<F, MT, NCH>;
    constexpr uint32_t S = SH::S, CB = SH::CB, WROW = SH::WROW, WI = SH::WI, WPW = SH::WPW, WBYTES = SH::WBYTES,
                       XI = SH::XI, XPW = SH::XPW, SLOT = SH::SLOT;
    static_assert(S >= 3, "ring of at least three chunks");
    constexpr uint32_t K = NCH * kStKC;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t M = p.M, N = p.N;
    const uint32_t n0 = blockIdx.x * kStCols;
    const uint32_t ncols = min((uint32_t)kStCols, N - n0);
    const uint32_t start = (blockIdx.x >> 3) % NCH;     // rotated K order per XCD slot
    uint8_t* const ring = smem + WBYTES;

    // W region: unit u (16 bytes) of column u / (WROW / 16); the pad unit and
    // the columns past N read as zeros.  Issued first: waiting for chunk 0
    // waits for it too.
    {
        const auto wr = make_rsrc(p.W + (size_t)n0 * CB, ncols * CB);
        constexpr uint32_t UPC = WROW / 16;
#pragma unroll
        for (uint32_t j = 0; j < WPW; j++) {
            const uint32_t i = (uint32_t)wave + kStWaves * j;
            const uint32_t u = i * 64 + lane, col = u / UPC, cu = u % UPC;
            const uint32_t off = (col < ncols && cu + 1 < UPC) ? col * CB + 16u * cu : kOOB;
            if (i < WI)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (__attribute__((address_space(3))) void*)(smem + i * 1024u),
                                                         16, off, 0, 0, 0);
        }
    }
    // X copies: copy i of a chunk holds rows 2i (lanes 0-31) and 2i + 1; lane
    // unit pu of row r is logical unit pu ^ (r mod 16) of the row's 512 bytes.
    // The chunk's K offset goes in soffset.
    const auto xr = make_rsrc(p.X, M * K * 2u);
    uint32_t xvo[XPW];
#pragma unroll
    for (uint32_t j = 0; j < XPW; j++) {
        const uint32_t i = (uint32_t)wave + kStWaves * j;
        const uint32_t row = 2u * i + ((uint32_t)lane >> 5);
        xvo[j] = row < M ? row * K * 2u + 16u * (((uint32_t)lane & 31u) ^ (row & 15u)) : kOOB;
    }
    auto kchunk = [&](uint32_t c) { return c + start < NCH ? c + start : c + start - NCH; };
    auto issue = [&](uint32_t c) {
        const uint32_t soff = kchunk(c) * kStKC * 2u;
        uint8_t* const dst = ring + (c % S) * SLOT;
#pragma unroll
        for (uint32_t j = 0; j < XPW; j++) {
            const uint32_t i = (uint32_t)wave + kStWaves * j;
            const uint32_t vo = xvo[j];  // a local: an array element as the operand made the host pass drop the stub
            if (i < XI)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(dst + i * 1024u),
                                                         16, vo, (int)soff, 0, 0);
        }
    };
    // Waves below XI % kStWaves issue XPW copies per chunk, the others XPW - 1
    // (XPW when kStWaves divides XI).
    constexpr uint32_t XREM = XI % kStWaves;
    const bool full = XREM == 0 || (uint32_t)wave < XREM;
    constexpr uint32_t PRE = S - 1 < NCH ? S - 1 : NCH;
#pragma unroll
    for (uint32_t c = 0; c < PRE; c++) issue(c);

    // LDS read offsets of this lane's B fragments (slot-relative) and weights
    const uint32_t gi = (uint32_t)wave;                 // group of the chunk this wave decodes
    // Elements 8g .. 8g + 7 of the group are 16-byte unit 4 gi + g of the row
    // (swizzled): 8 (or 16) lanes of one read pass hit 8 (16) distinct units.
    uint32_t xo[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const uint32_t m = 16u * t + r16;
        xo[t] = (m >> 1) * 1024u + (m & 1u) * 512u + 16u * ((4u * gi + (uint32_t)g) ^ (m & 15u));
    }
    const uint8_t* const strip = smem + (uint32_t)r16 * WROW;

    f4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f4_t{};
#pragma unroll
    for (uint32_t c = 0; c < NCH; c++) {
        // chunks issued after c: min(S - 2, NCH - 1 - c), a constant once unrolled
        constexpr uint32_t AMAX = S - 2;
        const uint32_t ahead = (NCH - 1 - c) < AMAX ? (NCH - 1 - c) : AMAX;
#define QR_ST_WAIT(A)                                                                    \
        if (ahead == (A)) {                                                              \
            if (full) wait_vmcnt<XPW * (A)>(); else wait_vmcnt<(XPW - 1) * (A)>();       \
        }
        QR_ST_WAIT(0) QR_ST_WAIT(1) QR_ST_WAIT(2) QR_ST_WAIT(3) QR_ST_WAIT(4) QR_ST_WAIT(5) QR_ST_WAIT(6)
#undef QR_ST_WAIT
        barrier_mem();
        if (c + S - 1 < NCH) issue(c + S - 1);
        const uint8_t* const xs = ring + (c % S) * SLOT;
        const uint32_t kb = kchunk(c) * 8u + gi;         // group within the column
        uint32_t raw[FR::kRaw];
        FR::load(strip, kb, g, raw);
        u4_t xf[MT];
#pragma unroll
        for (int t = 0; t < MT; t++)  // rows past M are zeros: their lanes skip the read
            xf[t] = 16u * t + r16 < M ? *reinterpret_cast<const u4_t*>(xs + xo[t]) : u4_t{0, 0, 0, 0};
        const h8_t a = FR::decode(raw, kb, g);
#pragma unroll
        for (int t = 0; t < MT; t++)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8_t, xf[t]), acc[t], 0, 0, 0);
    }

    // ---- the 8 group partials of every output through LDS, fixed order ----
    // red [gi][m][n] with row stride RS = 16 + 4 floats; acc[t] holds
    // n = 4g + i, m = 16 t + r16.
    constexpr int RS = kStCols + 4;
    constexpr int ROWS = MT * 16;
    float* red = reinterpret_cast<float*>(smem);
    barrier_mem();  // every wave is done reading W and the ring (all copies were waited for)
#pragma unroll
    for (int t = 0; t < MT; t++)
        *reinterpret_cast<f4_t*>(red + (gi * ROWS + 16 * t + r16) * RS + 4 * g) = acc[t];
    __syncthreads();
    for (uint32_t idx = tid; idx < M * kStCols; idx += kStThreads) {
        const uint32_t m = idx / kStCols, nl = idx % kStCols;
        if (nl >= ncols) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; w++) v += red[(w * ROWS + m) * RS + nl];
        const uint32_t n = n0 + nl;
        if (p.R) v += (float)p.R[(size_t)m * N + n];
        size_t o;
        if (p.head_D) {
            const uint32_t h = n / p.head_D, dd = n % p.head_D;
            o = ((size_t)h * M + m) * p.head_D + dd;
        } else {
            o = (size_t)m * N + n;
        }
        p.Y[o] = (_Float16)v;
    }
}

template <int F, int MT, int NCH>
static hipError_t launch_st(const GemmParams& p, hipStream_t st) {
    using SH = StShape<F, MT, NCH>;
    if constexpr (SH::S < 3) {
        return hipErrorInvalidValue;  // st_plan never picks a shape whose ring does not fit
    } else {
        auto kern = gemm_stream_kernel<F, MT, NCH>;
        if (p.K != NCH * kStKC || p.col_bytes != SH::CB) return hipErrorInvalidValue;
        static size_t attr[kMaxDevices] = {};
        hipError_t e = lds_limit_once((const void*)kern, SH::LDS, attr);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, dim3((p.N + kStCols - 1) / kStCols), dim3(kStThreads), SH::LDS, st, p);
        return hipGetLastError();
    }
}

template <int F, int NCH>
static hipError_t launch_st_m(const GemmParams& p, hipStream_t st) {
    switch ((p.M + 15) / 16) {
        case 1: return launch_st<F, 1, NCH>(p, st);
        case 2: return launch_st<F, 2, NCH>(p, st);
        case 3: return launch_st<F, 3, NCH>(p, st);
        case 4: return launch_st<F, 4, NCH>(p, st);
        default: return hipErrorInvalidValue;
    }
}

template <int F>
static hipError_t launch_st_k(const GemmParams& p, hipStream_t st) {
    switch (p.K / kStKC) {
        case 8: return launch_st_m<F, 8>(p, st);
        case 16: return launch_st_m<F, 16>(p, st);
        default: return hipErrorInvalidValue;
    }
}

// Ring depth of the shape a (format, M, K) takes, 0 when there is none.
static uint32_t st_slots(int f, uint32_t M, uint32_t K) {
    const uint32_t nch = K / kStKC, mt = (M + 15) / 16;
    if (K % kStKC || (nch != 8 && nch != 16) || mt < 1 || mt > 4) return 0;
#define QR_ST_S(FF, NN) (mt == 1 ? StShape<FF, 1, NN>::S : mt == 2 ? StShape<FF, 2, NN>::S : mt == 3 ? StShape<FF, 3, NN>::S : StShape<FF, 4, NN>::S)
#define QR_ST_SF(FF) (nch == 8 ? QR_ST_S(FF, 8) : QR_ST_S(FF, 16))
    switch (f) {
        case QUANT_Q4_0: return QR_ST_SF(QUANT_Q4_0);
        case QUANT_MLX_4BIT: return QR_ST_SF(QUANT_MLX_4BIT);
        case QUANT_Q4_K: return QR_ST_SF(QUANT_Q4_K);
        case QUANT_TERNARY_1_58: return QR_ST_SF(QUANT_TERNARY_1_58);
        case QUANT_MLX_4BIT_G64: return QR_ST_SF(QUANT_MLX_4BIT_G64);
        default: return 0;
    }
#undef QR_ST_SF
#undef QR_ST_S
}

// The single-kernel form when its grid of 16-column workgroups covers the
// 256 CUs without reading X from L2 more than twice per CU, K is 2048 or 4096,
// and LDS holds the weight strip and a ring of at least 3 chunks.
static bool st_plan(int f, uint32_t M, uint32_t N, uint32_t K) {
    if (M == 0 || M > 64) return false;
    const uint32_t groups = (N + kStCols - 1) / kStCols;
    if (groups < 256 || groups > 512) return false;
    return st_slots(f, M, K) >= 3;
}

static uint32_t group_bytes_rt(int f) {
    switch (f) {
        case QUANT_Q4_0: return GroupBytes<QUANT_Q4_0>::v;
        case QUANT_MLX_4BIT: return GroupBytes<QUANT_MLX_4BIT>::v;
        case QUANT_Q4_K: return GroupBytes<QUANT_Q4_K>::v;
        case QUANT_TERNARY_1_58: return GroupBytes<QUANT_TERNARY_1_58>::v;
        case QUANT_MLX_4BIT_G64: return GroupBytes<QUANT_MLX_4BIT_G64>::v;
        default: return 0;
    }
}

// Split selection: 4, 2 or 1 groups per wave (K range 1024, 512 or 256 per
// workgroup); the longest range that still gives >= 256 workgroups, fits LDS
// and needs at most 16 splits.
static bool sk_plan(int f, uint32_t M, uint32_t N, uint32_t K, uint32_t* ks_out, uint32_t* gpw_out) {
    const uint32_t gb = group_bytes_rt(f);
    if (!gb || M == 0 || M > 64 || K % 256) return false;
    const uint32_t groups = (N + kSkCols - 1) / kSkCols;
    const uint32_t ng = K / 32;
    for (uint32_t gpw : {4u, 2u, 1u}) {
        if (ng % (gpw * kSkWaves) || (gpw * kSkWaves * gb) % 16) continue;
        const uint32_t ks = ng / (gpw * kSkWaves);
        if (ks > 16) continue;
        if (groups * ks < 256 && gpw > 1) continue;
        if (sk_layout(M, gpw, gb).lds > kSkLdsMax) continue;
        *ks_out = ks;
        *gpw_out = gpw;
        return true;
    }
    return false;
}

size_t skinny_workspace_floats(uint32_t M, uint32_t N, uint32_t K) {
    uint32_t ks_max = 1;
    for (int f : {0, 1, 2, 3, (int)QUANT_MLX_4BIT_G64}) {
        uint32_t ks = 1, gpw = 1;
        if (st_plan(f, M, N, K)) continue;  // single kernel: no partials
        if (sk_plan(f, M, N, K, &ks, &gpw) && ks > ks_max) ks_max = ks;
    }
    return ks_max > 1 ? (size_t)ks_max * M * N : 0;
}

template <int F, int MT, int GPW>
static hipError_t launch_sk(const GemmParams& p, float* ws, uint32_t ks, hipStream_t st) {
    if constexpr ((GPW * kSkWaves * GroupBytes<F>::v) % 16 != 0) {
        return hipErrorInvalidValue;  // sk_plan never picks a strip that is not whole 16-byte chunks
    } else {
    auto kern = gemm_skinny_kernel<F, MT, GPW>;
    const uint32_t groups = (p.N + kSkCols - 1) / kSkCols;
    const size_t lds = sk_layout(p.M, GPW, GroupBytes<F>::v).lds;
    static size_t attr[kMaxDevices] = {};  // dynamic LDS limit set for this instantiation, per device
    hipError_t e = lds_limit_once((const void*)kern, lds, attr);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(groups, ks), dim3(kSkThreads), lds, st, p, ws, ks);
    e = hipGetLastError();
    if (e == hipSuccess && ks > 1) e = launch_splitk_reduce(ws, ks, p.M, p.N, false, p.R, p.Y, p.head_D, st);
    return e;
    }
}

template <int F, int MT>
static hipError_t launch_sk_g(const GemmParams& p, float* ws, uint32_t ks, uint32_t gpw, hipStream_t st) {
    switch (gpw) {
        case 1: return launch_sk<F, MT, 1>(p, ws, ks, st);
        case 2: return launch_sk<F, MT, 2>(p, ws, ks, st);
        case 4: return launch_sk<F, MT, 4>(p, ws, ks, st);
        default: return hipErrorInvalidValue;
    }
}

template <int F>
static hipError_t launch_sk_m(const GemmParams& p, float* ws, hipStream_t st) {
    if (st_plan(F, p.M, p.N, p.K)) return launch_st_k<F>(p, st);
    uint32_t ks = 0, gpw = 0;
    if (!sk_plan(F, p.M, p.N, p.K, &ks, &gpw)) return hipErrorInvalidValue;
    switch ((p.M + 15) / 16) {
        case 1: return launch_sk_g<F, 1>(p, ws, ks, gpw, st);
        case 2: return launch_sk_g<F, 2>(p, ws, ks, gpw, st);
        case 3: return launch_sk_g<F, 3>(p, ws, ks, gpw, st);
        case 4: return launch_sk_g<F, 4>(p, ws, ks, gpw, st);
        default: return hipErrorInvalidValue;
    }
}

bool skinny_supported(const GemmParams& p) {
    if (p.W2 || !((p.format >= 0 && p.format <= 3) || p.format == QUANT_MLX_4BIT_G64)) return false;
    if (p.col_bytes % 16) return false;
    uint32_t ks, gpw;
    return st_plan(p.format, p.M, p.N, p.K) || sk_plan(p.format, p.M, p.N, p.K, &ks, &gpw);
}

hipError_t launch_gemm_skinny(const GemmParams& p, float* ws, hipStream_t st) {
    switch (p.format) {
        case QUANT_Q4_0: return launch_sk_m<QUANT_Q4_0>(p, ws, st);
        case QUANT_MLX_4BIT: return launch_sk_m<QUANT_MLX_4BIT>(p, ws, st);
        case QUANT_Q4_K: return launch_sk_m<QUANT_Q4_K>(p, ws, st);
        case QUANT_TERNARY_1_58: return launch_sk_m<QUANT_TERNARY_1_58>(p, ws, st);
        case QUANT_MLX_4BIT_G64: return launch_sk_m<QUANT_MLX_4BIT_G64>(p, ws, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qr
