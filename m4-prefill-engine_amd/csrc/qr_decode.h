// qr_decode.h -- per-format weight decoders for gfx950.
//
// Each decoder turns one 32-element group of one output column into 32
// binary16 weights, packed as 16 half2 words (word p holds elements 2p, 2p+1);
// decode_half(h) produces words 8h .. 8h+7 (elements 16h .. 16h+15) alone.
// Every weight is the round-to-nearest-even binary16 of the exact value the
// reference's double-precision CPU gold computes (tests/e2e/cpu_gold_reference.h),
// so decoded tiles are bit-identical to the CPU unpack:
//   Q4_0     w = (q - 8) d          cpu_gold_reference.h:37-40
//   MLX_4BIT w = q d + bias         cpu_gold_reference.h:78-81
//   Q4_K     w = q (d sc) - dmin m  cpu_gold_reference.h:121-142
//   TERNARY  w = (c - 1) d          cpu_gold_reference.h:178-187 (code 3 -> +2d)
// Nibble order in the 4-bit formats: byte i low nibble -> element i, high
// nibble -> element i + 16, so half h of a group is the low (h = 0) or high
// (h = 1) nibbles of all 16 code bytes.
//
// Loads go through a buffer resource whose base is the tile's first column,
// so `col_off` is the byte offset of the column inside the tile.  The weight
// base must be 4-byte aligned (the host checks and re-stages otherwise).
// Out-of-range loads return zeros, which decode to zero weights.
#pragma once
#include "qr_device.h"
#include "qr_formats.h"

namespace qr {

template <int F> struct Decoder;

// --------------------------------------------------------------------------
// Q4_0: 18-byte blocks, only 2-byte aligned inside a column.  Five aligned
// dwords cover the block at either parity; the 16 code bytes are re-aligned
// with a byte funnel shift.  Weights: (q - 8) * d in binary16 (q - 8 exact, one
// rounding).  The GEMM kernels use decode_half_fast instead: fma(q, d, -8 d),
// also one rounding of the exact value, one instruction less per pair; it
// differs only in the sign of a zero weight (q = 8 with d < 0 gives +0, the
// CPU unpack -0), which changes no product sum.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_Q4_0> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 18;
    static constexpr int kRawWords = 5;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[5]) {
        const uint32_t a = (col_off + kb * 18u) & ~3u;
#pragma unroll
        for (int i = 0; i < 5; i++) raw[i] = ld_b32(r, a + 4u * i);
    }
    __device__ static uint32_t scale_bits(const uint32_t raw[5], uint32_t parity2) {
        return parity2 ? (raw[0] >> 16) : (raw[0] & 0xffffu);  // block at byte 2 of raw[0]?
    }
    // The lane's block starts at byte parity2 (0 or 2) of raw[0]; one byte
    // permute per word picks the code dword (bytes 2 .. 5, or 4 .. 7, of the
    // pair raw[i], raw[i + 1]) and the scale twice (d, d), with the selector
    // formed once per block instead of a select per word.
    __device__ static uint32_t code_sel(uint32_t parity2) { return 0x05040302u + parity2 * 0x01010101u; }
    __device__ static uint32_t codes(const uint32_t raw[5], uint32_t sel, int i) {
        return perm(raw[i + 1], raw[i], sel);
    }
    __device__ static uint32_t scale_pair(const uint32_t raw[5], uint32_t sel) {
        return perm(raw[0], raw[0], sel - 0x04040202u);  // bytes 0 1 0 1 or 2 3 2 3
    }
    // GEMM operand path: fma(q, d, -8 d) -- -8 d is exact and the fused op
    // rounds once.  Valid while -8 d is finite (|d| <= 8188); needs_exact()
    // flags the rest.  Zero weights come out +0 (see above).
    __device__ static void decode_half_fast(const uint32_t raw[5], uint32_t parity2, int h, uint32_t out[8]) {
        const uint32_t sel = code_sel(parity2);
        const h2_t d = as_h2(scale_pair(raw, sel));
        const h2_t m8 = {(_Float16)-8.0f, (_Float16)-8.0f};
        const h2_t c = d * m8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = codes(raw, sel, i);
            const uint32_t n = (h ? (q >> 4) : q) & 0x0f0f0f0fu;
            out[2 * i + 0] = as_u32(__builtin_elementwise_fma(code_pair<false>(n), d, c));
            out[2 * i + 1] = as_u32(__builtin_elementwise_fma(code_pair<true>(n), d, c));
        }
    }
    // Any scale: (q - 8) exact in binary16, one rounding in the product.
    __device__ static void decode_half_exact(const uint32_t raw[5], uint32_t parity2, int h, uint32_t out[8]) {
        const uint32_t sel = code_sel(parity2);
        const h2_t d = as_h2(scale_pair(raw, sel));
        const h2_t off = {(_Float16)8.0f, (_Float16)8.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = codes(raw, sel, i);
            const uint32_t n = (h ? (q >> 4) : q) & 0x0f0f0f0fu;
            out[2 * i + 0] = as_u32((code_pair<false>(n) - off) * d);
            out[2 * i + 1] = as_u32((code_pair<true>(n) - off) * d);
        }
    }
    __device__ static bool needs_exact(const uint32_t raw[5], uint32_t parity2) {
        return !(__builtin_fabsf(h2f(scale_bits(raw, parity2))) <= kQ4_0FastMaxScale);
    }
    __device__ static void decode_half(const uint32_t raw[5], uint32_t parity2, int h, uint32_t out[8]) {
        decode_half_exact(raw, parity2, h, out);
    }
    __device__ static uint32_t parity(uint32_t col_off, uint32_t kb) { return (col_off + kb * 18u) & 2u; }
};

// --------------------------------------------------------------------------
// MLX_4BIT: 20-byte blocks (dword aligned).  w = fma(q, d, bias) in binary16:
// q is exact, and the fused multiply-add rounds once.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_MLX_4BIT> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 20;
    static constexpr int kRawWords = 5;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[5]) {
        const uint32_t o = col_off + kb * 20u;
#pragma unroll
        for (int i = 0; i < 5; i++) raw[i] = ld_b32(r, o + 4u * i);
    }
    __device__ static void decode_half(const uint32_t raw[5], uint32_t, int h, uint32_t out[8]) {
        const uint32_t d16 = raw[0] & 0xffffu, b16 = raw[0] >> 16;
        const h2_t d = as_h2(d16 | (d16 << 16));
        const h2_t bias = as_h2(b16 | (b16 << 16));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = raw[i + 1];
            const uint32_t n = (h ? (q >> 4) : q) & 0x0f0f0f0fu;
            out[2 * i + 0] = as_u32(__builtin_elementwise_fma(code_pair<false>(n), d, bias));
            out[2 * i + 1] = as_u32(__builtin_elementwise_fma(code_pair<true>(n), d, bias));
        }
    }
    __device__ static uint32_t parity(uint32_t, uint32_t) { return 0; }
};

// --------------------------------------------------------------------------
// Q4_K: 144-byte super-blocks of 8 sub-blocks of 32.  Per sub-block the
// reference's 6-bit scale sc and min m (its own packing, cpu_gold_reference.h:
// 121-127).  A = d*sc and B = dmin*m are exact floats; q*A is exact.  When the
// binade gap between d and dmin is small (e_d - e_dmin <= 3 and
// e_dmin - e_d <= 7) the exact q*A - B has <= 24 significant bits, so one fp32
// fma is exact and a single conversion gives the RNE binary16; otherwise the
// exact-sum path (round-to-odd) is used, as a wave-uniform branch.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_Q4_K> {
    static constexpr int kBlockElems = 32;  // decode granularity (sub-block)
    static constexpr int kBlockBytes = 144; // per 256 elements
    static constexpr int kRawWords = 8;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[8]) {
        const uint32_t o = col_off + (kb >> 3) * 144u;
        const u4_t hd = ld_b128(r, o);
        const u4_t q = ld_b128(r, o + 16u + 16u * (kb & 7u));
        raw[0] = hd.x; raw[1] = hd.y; raw[2] = hd.z; raw[3] = hd.w;
        raw[4] = q.x; raw[5] = q.y; raw[6] = q.z; raw[7] = q.w;
    }
    __device__ static int binade(uint32_t h16) {
        const int e = (int)((h16 >> 10) & 0x1f);
        return (e < 1 ? 1 : e) - 15;
    }
    // A, B and the exactness flag of sub-block s from the header words.
    __device__ static void scales(const uint32_t raw[4], uint32_t s, float& A, float& B, bool& fast) {
        const uint32_t d16 = raw[0] & 0xffffu, dm16 = raw[0] >> 16;
        const uint64_t s07 = (uint64_t)raw[1] | ((uint64_t)raw[2] << 32);  // scales[0..7]
        const uint32_t scj = (uint32_t)(s07 >> (8u * s)) & 0xffu;
        const uint32_t sc = scj & 63u;
        const uint32_t lowm = (s < 4) ? ((raw[3] >> (8u * s)) & 0x0fu) : ((raw[3] >> (8u * (s - 4u) + 4u)) & 0x0fu);
        const uint32_t mn = lowm | ((scj >> 6) << 4);
        A = h2f(d16) * (float)sc;
        B = h2f(dm16) * (float)mn;
        const int gap = binade(d16) - binade(dm16);
        fast = (A == 0.0f) || (B == 0.0f) || (gap <= 3 && gap >= -7);
    }
    // Fast path only (caller has established that no lane needs the exact-sum path).
    __device__ static void decode_half_fast(const uint32_t raw[8], uint32_t s, int h, uint32_t out[8]) {
        float A, B;
        bool fast;
        scales(raw, s, A, B, fast);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t n = (h ? (raw[4 + i] >> 4) : raw[4 + i]) & 0x0f0f0f0fu;
            out[2 * i + 0] = affine_pair_exact(code_pair<false>(n), A, -B);
            out[2 * i + 1] = affine_pair_exact(code_pair<true>(n), A, -B);
        }
    }
    __device__ static bool needs_exact(const uint32_t raw[8], uint32_t s) {
        float A, B;
        bool fast;
        scales(raw, s, A, B, fast);
        return !fast;
    }
    __device__ static void decode_half(const uint32_t raw[8], uint32_t s, int h, uint32_t out[8]) {
        float A, B;
        bool fast;
        scales(raw, s, A, B, fast);
        if (__all(fast)) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t n = (h ? (raw[4 + i] >> 4) : raw[4 + i]) & 0x0f0f0f0fu;
                out[2 * i + 0] = affine_pair_exact(code_pair<false>(n), A, -B);
                out[2 * i + 1] = affine_pair_exact(code_pair<true>(n), A, -B);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t n = (h ? (raw[4 + i] >> 4) : raw[4 + i]) & 0x0f0f0f0fu;
                out[2 * i + 0] = affine_pair_any(code_pair<false>(n), A, -B, fast);
                out[2 * i + 1] = affine_pair_any(code_pair<true>(n), A, -B, fast);
            }
        }
    }
    __device__ static uint32_t parity(uint32_t, uint32_t kb) { return kb & 7u; }
};

// 16 two-bit codes of word q (element e at bits 2e, LSB first) as 8 binary16
// pairs (c - 1) d, code 3 giving +2d.  The four values are formed once, as
// the binary16 products {-1, 0} d and {1, 2} d (exact but for the overflow
// of 2d, which the CPU gold shares); each pair is then one byte-permute
// lookup into those 8 bytes, its selector (bytes 2c, 2c + 1 per element)
// built from the codes by one permute and one shift-or.  Shared by
// TERNARY_1_58 and PRISM_Q2_0.
__device__ __forceinline__ void two_bit_word(uint32_t q, uint32_t d16, uint32_t out[8]) {
    const h2_t d = as_h2(d16 | (d16 << 16));
    const uint32_t t01 = as_u32(h2_t{(_Float16)-1.0f, (_Float16)0.0f} * d);  // bytes 0-3: codes 0, 1
    const uint32_t t23 = as_u32(h2_t{(_Float16)1.0f, (_Float16)2.0f} * d);   // bytes 4-7: codes 2, 3
    const uint32_t ev = q & 0x33333333u;         // codes of even elements, one per nibble
    const uint32_t od = (q >> 2) & 0x33333333u;  // codes of odd elements
    const uint32_t ev_lo = ev & 0x0f0f0f0fu, ev_hi = (ev >> 4) & 0x0f0f0f0fu;
    const uint32_t od_lo = od & 0x0f0f0f0fu, od_hi = (od >> 4) & 0x0f0f0f0fu;
    // nibble j (elements 2j, 2j+1): j even -> byte j/2 of *_lo, j odd -> of *_hi
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uint32_t sel = 0x04040000u + 0x01010101u * (uint32_t)b;  // bytes {c_even, c_even, c_odd, c_odd}
        const uint32_t s0 = (perm(od_lo, ev_lo, sel) << 1) | 0x01000100u;  // nibble 2b
        const uint32_t s1 = (perm(od_hi, ev_hi, sel) << 1) | 0x01000100u;  // nibble 2b+1
        out[2 * b + 0] = perm(t23, t01, s0);
        out[2 * b + 1] = perm(t23, t01, s1);
    }
}

// --------------------------------------------------------------------------
// TERNARY_1_58: 12-byte blocks (dword aligned); qs[0] holds elements 0..15,
// qs[1] elements 16..31, two bits each, LSB first.  w = (c - 1) d
// in binary16: exact for every code, code 3 giving +2d as the CPU gold does.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_TERNARY_1_58> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 12;
    static constexpr int kRawWords = 3;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[3]) {
        const uint32_t o = col_off + kb * 12u;
#pragma unroll
        for (int i = 0; i < 3; i++) raw[i] = ld_b32(r, o + 4u * i);
    }
    __device__ static void decode_half(const uint32_t raw[3], uint32_t, int h, uint32_t out[8]) {
        two_bit_word(h ? raw[2] : raw[1], raw[0] & 0xffffu, out);
    }
    __device__ static uint32_t parity(uint32_t, uint32_t) { return 0; }
};

// --------------------------------------------------------------------------
// Formats whose CPU gold forms each weight with double-precision roundings
// (VAR_RATE_AFFINE, EXL3): the weight is computed here with the same double
// operations -- every product involved is exact in double, so fused and
// separate multiply-add round identically -- and then rounded ONCE to
// binary16: the double is narrowed to float with round-to-odd (>= 2 spare
// bits), whose RNE conversion to binary16 equals RNE of the double.
// --------------------------------------------------------------------------
__device__ __forceinline__ uint32_t rne16_from_f64(double w) {
    const float f = (float)w;
    uint32_t bits = f32_bits(f);
    const double back = (double)f;
    if (back != w) {
        const bool away = __builtin_fabs(back) > __builtin_fabs(w);
        bits = (away ? bits - 1u : bits) | 1u;
    }
    return f2h_bits(bits_f32(bits));
}

// Code j (0..31) of an LSB-first bit stream of B-bit codes held in `q`.
// (j is a compile-time constant after unrolling: the second word is read only
// when the code straddles a word boundary.)
template <int B>
__device__ __forceinline__ uint32_t stream_code(const uint32_t* q, int j) {
    const int bit = j * B, w = bit >> 5, sh = bit & 31;
    uint32_t v = q[w] >> sh;
    if (sh + B > 32) v |= q[w + 1] << (32 - sh);
    return v & ((1u << B) - 1u);
}

// --------------------------------------------------------------------------
// VAR_RATE_AFFINE: 160-byte super-blocks of 8 sub-blocks of 32
// (cpu_gold_reference.h:212-323).  Sub-block s: scale S = d sc / 16, bias
// B = bias + d (bi - 128) / 16; mode bits 0..2 = code depth (3 and 5: LSB-first
// bit streams of 12 / 20 bytes; anything else: 4-bit, byte i low nibble ->
// code i, high -> code i + 16), bits 3..4 = order (1: code j multiplies
// element ((j & 1) << 4) | (j >> 1); 2: element 31 - j; else element j).
// w = (q - 2^(depth-1)) S + B.  Raw words: header dwords 0..6 (d | bias,
// scales, biases, modes), then 5 code dwords from byte 32 + offset[s].
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_VAR_RATE_AFFINE> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 160;
    static constexpr int kRawWords = 12;
    // sub-block payload offsets {0, 12, 24, 40, 56, 72, 88, 108}, one per byte
    static constexpr uint64_t kOffsets = 0x6C58483828180C00ull;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[12]) {
        const uint32_t o = col_off + (kb >> 3) * 160u;
        const u4_t h0 = ld_b128(r, o);
        const u4_t h1 = ld_b128(r, o + 16u);
        raw[0] = h0.x; raw[1] = h0.y; raw[2] = h0.z; raw[3] = h0.w;
        raw[4] = h1.x; raw[5] = h1.y; raw[6] = h1.z;
        const uint32_t q = o + 32u + (uint32_t)((kOffsets >> (8u * (kb & 7u))) & 0xffu);  // 4-byte aligned
#pragma unroll
        for (int i = 0; i < 5; i++) raw[7 + i] = ld_b32(r, q + 4u * i);
    }
    __device__ static uint32_t byte_of(const uint32_t* w, uint32_t i) { return (w[i >> 2] >> (8u * (i & 3u))) & 0xffu; }
    // code j of the sub-block at depth 3, 5 or 4 (j compile-time after unrolling)
    __device__ __forceinline__ static uint32_t code(const uint32_t* q, bool d3, bool d5, int j) {
        const uint32_t c4 = j < 16 ? (byte_of(q, (uint32_t)j) & 15u) : (byte_of(q, (uint32_t)(j - 16)) >> 4);
        return d3 ? stream_code<3>(q, j) : (d5 ? stream_code<5>(q, j) : c4);
    }
    __device__ __forceinline__ static void decode_half(const uint32_t raw[12], uint32_t s, int h, uint32_t out[8]) {
        const double d = (double)h2f(raw[0] & 0xffffu), bias = (double)h2f(raw[0] >> 16);
        const uint32_t sc = (uint32_t)((((uint64_t)raw[2] << 32) | raw[1]) >> (8u * s)) & 0xffu;
        const uint32_t bi = (uint32_t)((((uint64_t)raw[4] << 32) | raw[3]) >> (8u * s)) & 0xffu;
        const uint32_t mode = (uint32_t)((((uint64_t)raw[6] << 32) | raw[5]) >> (8u * s)) & 0xffu;
        const double S = d * (double)sc * 0.0625;
        const double B = bias + d * ((double)bi - 128.0) * 0.0625;
        const uint32_t depth = mode & 7u, order = (mode >> 3) & 3u;
        const uint32_t* q = raw + 7;
        const bool d3 = depth == 3u, d5 = depth == 5u;
        const double zero = d3 ? 4.0 : (d5 ? 16.0 : 8.0);
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            uint32_t hw[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int p = 16 * h + e + t;                      // element (activation) index
                const int j1 = p < 16 ? 2 * p : 2 * (p - 16) + 1;  // order 1: code that lands on p
                const uint32_t c = order == 1u ? code(q, d3, d5, j1) : (order == 2u ? code(q, d3, d5, 31 - p) : code(q, d3, d5, p));
                hw[t] = rne16_from_f64(__builtin_fma((double)c - zero, S, B));
            }
            out[e >> 1] = hw[0] | (hw[1] << 16);
        }
    }
    __device__ static uint32_t parity(uint32_t, uint32_t kb) { return kb & 7u; }
};

// --------------------------------------------------------------------------
// EXL3: 144-byte super-blocks of 8 sub-blocks of 32 (cpu_gold_reference.h:
// 345-392).  Sub-block s: S = d sc / 64, R = d (res - 128) / 128; 3-bit codes
// q (LSB-first stream, 12 bytes at byte 48 + 12 s); int8 codebook cb[16];
// w = (bias + S cb[q]) + R cb[q + 8].  Raw words: header dwords 0..8 (d | bias,
// scales, residuals, codebook), then the 3 code dwords.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_EXL3> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 144;
    static constexpr int kRawWords = 12;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[12]) {
        const uint32_t o = col_off + (kb >> 3) * 144u;
        const u4_t h0 = ld_b128(r, o);
        const u4_t h1 = ld_b128(r, o + 16u);
        raw[0] = h0.x; raw[1] = h0.y; raw[2] = h0.z; raw[3] = h0.w;
        raw[4] = h1.x; raw[5] = h1.y; raw[6] = h1.z; raw[7] = h1.w;
        raw[8] = ld_b32(r, o + 32u);
        const uint32_t q = o + 48u + 12u * (kb & 7u);
        raw[9] = ld_b32(r, q);
        raw[10] = ld_b32(r, q + 4u);
        raw[11] = ld_b32(r, q + 8u);
    }
    __device__ __forceinline__ static void decode_half(const uint32_t raw[12], uint32_t s, int h, uint32_t out[8]) {
        const double d = (double)h2f(raw[0] & 0xffffu), bias = (double)h2f(raw[0] >> 16);
        const uint32_t sc = (uint32_t)((((uint64_t)raw[2] << 32) | raw[1]) >> (8u * s)) & 0xffu;
        const uint32_t rs = (uint32_t)((((uint64_t)raw[4] << 32) | raw[3]) >> (8u * s)) & 0xffu;
        const double S = d * (double)sc * 0.015625;
        const double R = d * ((double)rs - 128.0) * 0.0078125;
        // codebook bytes 20..35 = raw[5] .. raw[8]: base cb[0..7] in raw[5], raw[6],
        // residual cb[8..15] in raw[7], raw[8]
        const uint32_t* q = raw + 9;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            uint32_t hw[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t code = stream_code<3>(q, 16 * h + e + t);
                const int cb0 = (int)(int8_t)(perm(raw[6], raw[5], code) & 0xffu);
                const int cb1 = (int)(int8_t)(perm(raw[8], raw[7], code) & 0xffu);
                hw[t] = rne16_from_f64(__builtin_fma(R, (double)cb1, __builtin_fma(S, (double)cb0, bias)));
            }
            out[e >> 1] = hw[0] | (hw[1] << 16);
        }
    }
    __device__ static uint32_t parity(uint32_t, uint32_t kb) { return kb & 7u; }
};

// --------------------------------------------------------------------------
// PRISM_Q2_0: 34-byte blocks of 128 elements {f16 d; u8 qs[32]}, four 2-bit
// codes per byte LSB first, element 4 i + j at bits 2 j of qs[i]
// (cpu_gold_reference.h:418-430; quant_router_kernels.metal:414-436).  Group
// kb is sub-block s = kb % 4 of block kb / 4: code bytes 8 s .. 8 s + 7, the
// same bit order as a ternary code word, so w = (c - 1) d with code 3 -> +2d
// (the gold and the reference's PRISM kernel agree on it).  Blocks are only
// 2-byte aligned: three aligned dwords cover the 8 code bytes at either
// parity, plus the dword holding d.  parity() packs the block's byte parity
// (bit 1) and s (bits 2..3).
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_PRISM_Q2_0> {
    static constexpr int kBlockElems = 32;   // decode granularity (sub-block)
    static constexpr int kBlockBytes = 34;   // per 128 elements
    static constexpr int kRawWords = 4;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[4]) {
        const uint32_t b = col_off + (kb >> 2) * 34u;
        const uint32_t c = (b + 2u + 8u * (kb & 3u)) & ~3u;
        raw[0] = ld_b32(r, b & ~3u);
        raw[1] = ld_b32(r, c);
        raw[2] = ld_b32(r, c + 4u);
        raw[3] = ld_b32(r, c + 8u);
    }
    __device__ static void decode_half(const uint32_t raw[4], uint32_t par, int h, uint32_t out[8]) {
        // block at byte 0 of its dword: d low, codes start at byte 2 of raw[1]
        const bool lo = (par & 2u) == 0;
        const uint32_t d16 = lo ? (raw[0] & 0xffffu) : (raw[0] >> 16);
        const uint32_t q = lo ? __builtin_amdgcn_alignbyte(raw[2 + h], raw[1 + h], 2) : raw[1 + h];
        two_bit_word(q, d16, out);
    }
    __device__ static uint32_t parity(uint32_t col_off, uint32_t kb) {
        return ((col_off + (kb >> 2) * 34u) & 2u) | ((kb & 3u) << 2);
    }
};

// --------------------------------------------------------------------------
// Q8_0 weights: 34-byte blocks {f16 d; i8 qs[32]}, w = q d (the registry's
// quant_router_gemm_q8_0_64x64, quant_registry.mm:153, a kernel the reference
// never wrote; the block is the KV-cache block of brick4_attn_bench.mm:57-65).
// q is exact in binary16 (magic exponent: 1024 + (q + 128) - 1152) and the
// product rounds once.  Nine aligned dwords cover the block at either parity.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_Q8_0> {
    static constexpr int kBlockElems = 32;
    static constexpr int kBlockBytes = 34;
    static constexpr int kRawWords = 9;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[9]) {
        const uint32_t a = (col_off + kb * 34u) & ~3u;
#pragma unroll
        for (int i = 0; i < 9; i++) raw[i] = ld_b32(r, a + 4u * i);
    }
    __device__ static void decode_half(const uint32_t raw[9], uint32_t par, int h, uint32_t out[8]) {
        const bool lo = par == 0u;  // block at byte 0 of raw[0]: codes from byte 2
        const uint32_t d16 = lo ? (raw[0] & 0xffffu) : (raw[0] >> 16);
        const h2_t d = as_h2(d16 | (d16 << 16));
        const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int w = 4 * h + i;  // code word: elements 4w .. 4w + 3
            const uint32_t q = (lo ? __builtin_amdgcn_alignbyte(raw[w + 1], raw[w], 2) : raw[w + 1]) ^ 0x80808080u;
            out[2 * i + 0] = as_u32((as_h2(nib_pair_lo(q)) - off) * d);
            out[2 * i + 1] = as_u32((as_h2(nib_pair_hi(q)) - off) * d);
        }
    }
    __device__ static uint32_t parity(uint32_t col_off, uint32_t kb) { return (col_off + kb * 34u) & 2u; }
};

// --------------------------------------------------------------------------
// MLX_4BIT_G64: 36-byte blocks of 64 elements (dword aligned): fp16 scale and
// bias, then eight code words, element 8j + i in bits 4i of word j (MLX's
// packing).  Decode group kb = half kb % 2 of block kb / 2, i.e. code words
// 4 (kb % 2) .. + 3; w = fma(q, scale, bias) in binary16, one rounding, as
// MLX_4BIT.  A code word's low and high nibbles are split into two byte
// vectors and interleaved back into element order with two byte permutes.
// --------------------------------------------------------------------------
template <> struct Decoder<QUANT_MLX_4BIT_G64> {
    static constexpr int kBlockElems = 32;  // decode granularity (half block)
    static constexpr int kBlockBytes = 36;  // per 64 elements
    static constexpr int kRawWords = 5;
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t col_off, uint32_t kb, uint32_t raw[5]) {
        const uint32_t o = col_off + (kb >> 1) * 36u;
        raw[0] = ld_b32(r, o);
        const uint32_t c = o + 4u + 16u * (kb & 1u);
#pragma unroll
        for (int i = 0; i < 4; i++) raw[i + 1] = ld_b32(r, c + 4u * i);
    }
    // bytes {c0, c1, c2, c3} and {c4, c5, c6, c7} of code word w
    __device__ static void codes8(uint32_t w, uint32_t& a, uint32_t& b) {
        const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
        a = perm(hi, lo, 0x05010400u);
        b = perm(hi, lo, 0x07030602u);
    }
    __device__ static void decode_half(const uint32_t raw[5], uint32_t, int h, uint32_t out[8]) {
        const uint32_t d16 = raw[0] & 0xffffu, b16 = raw[0] >> 16;
        const h2_t d = as_h2(d16 | (d16 << 16));
        const h2_t bias = as_h2(b16 | (b16 << 16));
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint32_t a, b;
            codes8(raw[1 + 2 * h + i], a, b);
            out[4 * i + 0] = as_u32(__builtin_elementwise_fma(code_pair<false>(a), d, bias));
            out[4 * i + 1] = as_u32(__builtin_elementwise_fma(code_pair<true>(a), d, bias));
            out[4 * i + 2] = as_u32(__builtin_elementwise_fma(code_pair<false>(b), d, bias));
            out[4 * i + 3] = as_u32(__builtin_elementwise_fma(code_pair<true>(b), d, bias));
        }
    }
    __device__ static uint32_t parity(uint32_t, uint32_t) { return 0; }
};

// Branch-free half-group decode for pipelined callers: bit-exact whenever no
// lane of the wave has needs_exact() true for its group (Q4_K and Q4_0 have a
// slow path; callers check and re-decode with decode_group otherwise).
template <int F>
__device__ __forceinline__ void decode_half_fast(const uint32_t* raw, uint32_t parity, int h, uint32_t out[8]) {
    if constexpr (F == QUANT_Q4_K || F == QUANT_Q4_0) Decoder<F>::decode_half_fast(raw, parity, h, out);
    else Decoder<F>::decode_half(raw, parity, h, out);
}
template <int F>
__device__ __forceinline__ bool needs_exact(const uint32_t* raw, uint32_t parity) {
    if constexpr (F == QUANT_Q4_K || F == QUANT_Q4_0) return Decoder<F>::needs_exact(raw, parity);
    else return false;
}

// Whole group: words 0..15.
template <int F>
__device__ __forceinline__ void decode_group(const uint32_t* raw, uint32_t parity, uint32_t out[16]) {
    Decoder<F>::decode_half(raw, parity, 0, out);
    Decoder<F>::decode_half(raw, parity, 1, out + 8);
}

}  // namespace qr
