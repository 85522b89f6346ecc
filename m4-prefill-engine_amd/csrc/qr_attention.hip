// qr_attention.hip -- Q8_0 KV-cache quantization and causal flash attention
// over the Q8_0 cache on gfx950.
//
// Replaces quantize_kv_to_q8_0 (unified_kernels.metal:118-145) and
// flash_attn_mma_64x64_q8_0_impl<D> (brick4_attn_kernels.metal:572-881).
//
//  * The Q8_0 cache is dequantized once per call into an fp16 cache (K' rows,
//    V' transposed), each value the reference's half(q * half(d))
//    (brick4_attn_bench.mm:57-65), so query tiles stage K/V tiles with plain
//    copies instead of decoding them again per query tile.
//  * Each wave owns 32 queries and computes S^T = K . Q^T with
//    v_mfma_f32_32x32x16_f16, so a lane owns ONE query column: the softmax
//    row statistics are lane-local over its 16 accumulator rows plus one
//    exchange with the partner lane (l ^ 32) -- no 32-lane reduction trees.
//  * P stays in registers: the S^T accumulator of a lane already holds the
//    8 keys that lane must supply as the B operand of O^T = V^T . P^T, given
//    the matching key order in the V^T A-operand reads (two ds_read_b64).
//  * fp32 running max / sum / output accumulators (the reference keeps
//    S, P and O in half); the output is rounded to fp16 once.
#include <type_traits>

#include "qr_device.h"
#include "qr_kernels.h"

namespace qr {

// --------------------------------------------------------------------------
// Q8_0 quantization: per 32 values amax in fp32, d = amax / 127 (IEEE
// division), stored as half(d); codes q = round(x * (1/d)) (half away from
// zero) with the UNROUNDED d, clamped to [-128, 127] (unified_kernels.metal:
// 118-145).  One thread per block.
// --------------------------------------------------------------------------
// One block: x[32] -> half(d) bits and 16 code words (two int8 codes each).
__device__ __forceinline__ void quantize_block_q8_0(const float x[32], uint32_t& d16, uint32_t codes[16]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    d16 = f2h_bits(d);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        int q0 = (int)__builtin_roundf(x[2 * i] * id);
        int q1 = (int)__builtin_roundf(x[2 * i + 1] * id);
        q0 = q0 < -128 ? -128 : (q0 > 127 ? 127 : q0);
        q1 = q1 < -128 ? -128 : (q1 > 127 ? 127 : q1);
        codes[i] = (uint32_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

__device__ __forceinline__ void load_block_f16(const _Float16* src, float x[32]) {
    const u4_t* s = reinterpret_cast<const u4_t*>(src);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u4_t v = s[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            x[8 * i + 2 * k] = h2f(w[k] & 0xffffu);
            x[8 * i + 2 * k + 1] = h2f(w[k] >> 16);
        }
    }
}

__global__ void __launch_bounds__(256) quantize_q8_0_kernel(const _Float16* src, uint8_t* dst, size_t nblocks) {
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    float x[32];
    load_block_f16(src + b * 32, x);
    uint32_t d16, codes[16];
    quantize_block_q8_0(x, d16, codes);
    uint16_t* o16 = reinterpret_cast<uint16_t*>(dst + b * 34);  // 34-byte blocks are 2-byte aligned
    o16[0] = (uint16_t)d16;
#pragma unroll
    for (int i = 0; i < 16; i++) o16[1 + i] = (uint16_t)codes[i];
}

hipError_t launch_quantize_q8_0(const _Float16* src, uint8_t* dst, size_t nblocks, hipStream_t st) {
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, st, src, dst,
                       nblocks);
    return hipGetLastError();
}

// --------------------------------------------------------------------------
// Flash attention
// --------------------------------------------------------------------------
constexpr int kBQ = 128;      // queries per query tile
constexpr int kBKV = 64;      // keys per tile of the cache pass; the fp16 cache pads M to a multiple
// The attention kernel reads a dequantized fp16 working copy of the cache: K'
// [H, Mp, D] (row-major) and V'^T [H, D, Mp] (keys contiguous per dim), Mp = M
// rounded up to whole 64-key tiles, so its LDS tiles are plain 16-byte copies.

// Two Q8_0 codes of bytes 0, 1 (HI = false) or 2, 3 (HI = true) of a code word
// times d: the code plus 128 becomes the binary16 1024 + 128 + q through the
// magic exponent (exact), 1152 is subtracted (exact) and the product rounds
// once -- the reference's half(q * d) (brick4_attn_bench.mm:57-65).
template <bool HI>
__device__ __forceinline__ uint32_t q8_pair(uint32_t codes, h2_t d) {
    const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t u = codes ^ 0x80808080u;  // two's complement byte -> q + 128
    return as_u32((as_h2(HI ? nib_pair_hi(u) : nib_pair_lo(u)) - off) * d);
}

// Dequantized fp16 cache for the attention kernel, one workgroup per 64-key
// tile of one head.  FROM_Q8: from Q8_0 blocks (half(q * half(d)), the
// reference's dequantizer, brick4_attn_bench.mm:57-65); otherwise from fp16
// K / V through the same quantize-then-dequantize arithmetic as
// quantize_q8_0_kernel + the Q8_0 path (bit-identical values), also writing
// the Q8_0 blocks themselves to Kq / Vq when those are given -- the layer's
// Q8_0 KV cache, produced in the same pass.  Every output goes through LDS so
// it leaves in contiguous runs: K units (one key's block) fill the tile's K'
// rows (one contiguous 64-key run of K'); V units (a key pair's blocks) write
// {V[k][d], V[k+1][d]} words into a tile [d][key] whose rows leave as 128-byte
// runs of V'^T; the Q8_0 blocks of the tile's keys (contiguous in the cache)
// leave as dword runs.  Keys M .. Mp - 1 are zero.
template <bool FROM_Q8>
__device__ __forceinline__ void prep_block(const void* src, size_t blk, uint32_t w[16], uint8_t* q8out) {
    uint32_t d16, codes[8];  // code word c: codes of elements 4c .. 4c + 3
    if constexpr (FROM_Q8) {
        // 34-byte blocks are 2-byte aligned.  From the aligned dword at or
        // below the block, eight dwords plus the next two bytes (block at a
        // dword boundary) or nine dwords (block at 2 mod 4) cover it exactly,
        // so nothing past the block's last byte is read.
        const size_t o = blk * 34;
        const uint8_t* base = static_cast<const uint8_t*>(src) + (o & ~(size_t)3);
        const uint32_t* q = reinterpret_cast<const uint32_t*>(base);
        const bool par = (o & 2u) != 0;
        uint32_t raw[9];
#pragma unroll
        for (int i = 0; i < 8; i++) raw[i] = q[i];
        raw[8] = par ? q[8] : (uint32_t)*reinterpret_cast<const uint16_t*>(base + 32);
        d16 = par ? (raw[0] >> 16) : (raw[0] & 0xffffu);
#pragma unroll
        for (int c = 0; c < 8; c++) codes[c] = par ? raw[c + 1] : __builtin_amdgcn_alignbyte(raw[c + 1], raw[c], 2);
    } else {
        float x[32];
        load_block_f16(static_cast<const _Float16*>(src) + blk * 32, x);
        uint32_t c16[16];
        quantize_block_q8_0(x, d16, c16);
#pragma unroll
        for (int c = 0; c < 8; c++) codes[c] = c16[2 * c] | (c16[2 * c + 1] << 16);
        if (q8out) {  // this block's 34 bytes (2-byte aligned)
            uint16_t* o16 = reinterpret_cast<uint16_t*>(q8out);
            o16[0] = (uint16_t)d16;
#pragma unroll
            for (int i = 0; i < 16; i++) o16[1 + i] = (uint16_t)c16[i];
        }
    }
    const h2_t d = as_h2(d16 | (d16 << 16));
#pragma unroll
    for (int c = 0; c < 8; c++) {
        w[2 * c] = q8_pair<false>(codes[c], d);
        w[2 * c + 1] = q8_pair<true>(codes[c], d);
    }
}

template <int D, bool FROM_Q8>
__global__ void __launch_bounds__(256) kv_prep_kernel(const void* Ksrc, const void* Vsrc, _Float16* Kf, _Float16* Vtf,
                                                      uint8_t* Kq, uint8_t* Vq, uint32_t M, uint32_t Mp) {
    constexpr int NB = D / 32;            // blocks per key
    constexpr int TR = kBKV + 8;          // LDS row (halfs) of the transposed tile
    constexpr int KU = kBKV * NB, VU = (kBKV / 2) * NB;
    __shared__ __attribute__((aligned(16))) _Float16 T[D * TR];
    constexpr int KR = D + 8;  // LDS row (halfs) of the K' tile
    __shared__ __attribute__((aligned(16))) _Float16 KS[kBKV * KR];
    // the tile's Q8_0 blocks (from fp16 input, when the cache is wanted):
    // keys k0 .. k0 + 63 of K, then of V, 34-byte blocks back to back
    constexpr int QB = kBKV * NB * 34;
    __shared__ __attribute__((aligned(16))) uint8_t QS[FROM_Q8 ? 4 : 2 * QB];
    const int tid = threadIdx.x;
    const uint32_t k0 = blockIdx.x * kBKV, hk = blockIdx.y;
    const size_t head_blocks = (size_t)M * NB, head_dst = (size_t)Mp * D;
    for (int u = tid; u < KU + VU; u += 256) {
        if (u < KU) {
            const int key = u % kBKV, db = u / kBKV;
            const uint32_t gk = k0 + key;
            uint32_t w[16] = {};
            if (gk < M)
                prep_block<FROM_Q8>(Ksrc, hk * head_blocks + (size_t)gk * NB + db, w,
                                    (!FROM_Q8 && Kq) ? QS + (key * NB + db) * 34 : nullptr);
            u4_t* dst = reinterpret_cast<u4_t*>(KS + key * KR + db * 32);
#pragma unroll
            for (int c = 0; c < 4; c++) dst[c] = u4_t{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
        } else {
            const int v = u - KU;
            const int kp = v % (kBKV / 2), db = v / (kBKV / 2);
            uint32_t w[2][16] = {};
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t gk = k0 + 2 * kp + e;
                if (gk < M)
                    prep_block<FROM_Q8>(Vsrc, hk * head_blocks + (size_t)gk * NB + db, w[e],
                                        (!FROM_Q8 && Vq) ? QS + QB + ((2 * kp + e) * NB + db) * 34 : nullptr);
            }
            uint32_t* t32 = reinterpret_cast<uint32_t*>(T);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int dd = db * 32 + 2 * i;
                t32[(dd * TR) / 2 + kp] = perm(w[1][i], w[0][i], 0x05040100u);
                t32[((dd + 1) * TR) / 2 + kp] = perm(w[1][i], w[0][i], 0x07060302u);
            }
        }
    }
    __syncthreads();
    // streaming (non-temporal) stores: the working copy is written once and
    // read by the next kernel; measured 11.2 -> 9.9 us (from Q8_0) and 10.5 ->
    // 9.5 us (from fp16) at H = 32, M = 2048, D = 64
    for (int c = tid; c < D * 8; c += 256) {
        const int d = c / 8, kc = c % 8;
        __builtin_nontemporal_store(*reinterpret_cast<const u4_t*>(T + d * TR + kc * 8),
                                    reinterpret_cast<u4_t*>(Vtf + hk * head_dst + (size_t)d * Mp + k0 + kc * 8));
    }
    for (int c = tid; c < kBKV * D / 8; c += 256) {  // the K' tile is one contiguous run
        const int key = c / (D / 8), kc = c % (D / 8);
        __builtin_nontemporal_store(*reinterpret_cast<const u4_t*>(KS + key * KR + kc * 8),
                                    reinterpret_cast<u4_t*>(Kf + hk * head_dst + (size_t)k0 * D + (size_t)c * 8));
    }
    if constexpr (!FROM_Q8) {
        if (Kq) {  // the tile's blocks are one contiguous run of the cache (a multiple of 4 bytes)
            const uint32_t nkeys = min((uint32_t)kBKV, M - k0);
            const size_t first = (hk * head_blocks + (size_t)k0 * NB) * 34;
            if (((reinterpret_cast<uintptr_t>(Kq) | reinterpret_cast<uintptr_t>(Vq)) & 3u) == 0) {
                const int ndw = (int)(nkeys * NB * 34 / 4);
                uint32_t* kd = reinterpret_cast<uint32_t*>(Kq + first);
                uint32_t* vd = reinterpret_cast<uint32_t*>(Vq + first);
                const uint32_t* ks = reinterpret_cast<const uint32_t*>(QS);
                const uint32_t* vs = reinterpret_cast<const uint32_t*>(QS + QB);
                for (int i = tid; i < ndw; i += 256) {
                    kd[i] = ks[i];
                    vd[i] = vs[i];
                }
            } else {  // caches only 2-byte aligned
                const int nh = (int)(nkeys * NB * 17);
                uint16_t* kd = reinterpret_cast<uint16_t*>(Kq + first);
                uint16_t* vd = reinterpret_cast<uint16_t*>(Vq + first);
                const uint16_t* ks = reinterpret_cast<const uint16_t*>(QS);
                const uint16_t* vs = reinterpret_cast<const uint16_t*>(QS + QB);
                for (int i = tid; i < nh; i += 256) {
                    kd[i] = ks[i];
                    vd[i] = vs[i];
                }
            }
        }
    }
}

// --------------------------------------------------------------------------
// Software-pipelined causal attention over the fp16 cache, with the
// query-tile pairing that balances the causal work: one workgroup per (light,
// heavy) pair of 128-query tiles -- a and qtiles - 1 - a -- so every
// workgroup carries the same work.  A key tile is 32-key units (four at D =
// 64, two at D = 128); units whose keys all lie above a wave's diagonal are
// skipped.
//
// D = 64 (NG = 2, 8 waves, two per SIMD): group 0 takes the light tile's
// queries and group 1 the heavy tile's on the key tiles both need; the heavy
// tile's remaining key tiles go in pairs, one tile of a pair per group (a last
// odd tile split two units per group), and group 0's partial softmax state is
// merged into group 1's at the end.
// D = 128 (NG = 1, 4 waves, one per SIMD, so a wave has the registers for the
// 32 x 128 output tile and both fragment sets): the light tile's key tiles,
// then the heavy tile's, as one stream, two tiles per barrier.
//
// Pipelining: while the softmax of unit u runs on the VALU, the S^T = K . Q^T
// MFMAs of unit u + 1 and the O^T += V^T . P^T MFMAs of unit u are issued from
// the same fenced instruction sequence, so the matrix pipe and the vector ALU
// work side by side inside every wave.  K/V tiles sit in a 4-deep LDS ring
// (tiles t and t + 1 read, the look-ahead S reading ahead where that tile is
// already visible, tiles t + 2 and t + 3 being written).  Arithmetic per
// unit: log2-unit softmax with the scale folded into one fma, a lazily moved
// reference point (threshold 2^8, decided per lane half, the halves combined
// only when it moves), fp32 state, P rounded to fp16 for the MFMA and for the
// row sums.
// --------------------------------------------------------------------------
// keys per tile of the pipelined kernel: 128 at D = 64, 64 at D = 128 (the
// 4-deep ring of K and V^T tiles then fits the LDS at either width)
constexpr int pipe_keys(int D) { return D == 64 ? 128 : 64; }
constexpr int kPVPad = 4;  // halfs of padding per V^T row of its LDS tiles

template <int D, int NG>  // NG: wave groups of 4 (2: the pair schedule; 1: the two tiles one after the other)
__global__ void __launch_bounds__(256 * NG) flash_attn_pipe_kernel(AttnParams p) {
    static_assert(D == 64 || D == 128, "chunk schedules written for D = 64 and D = 128");
    constexpr int kPKV = pipe_keys(D), UPT = kPKV / 32;  // units (32 keys) per tile
    // V^T rows of kPKV + 4 halfs (66 or 34 dwords): the fragment reads of
    // lanes j and j + 16 land 32 banks apart (a 68-dword row put them on the
    // same banks)
    constexpr int KROW = D + 8, VROW = kPKV + kPVPad, DT = D / 32;
    constexpr int NT = 256 * NG;
    constexpr int KT = kPKV * KROW, VT = D * VROW, TILE = KT + VT;
    constexpr int NBUF = 4;
    constexpr int KCH = kPKV * (D / 8) / NT, VCH = D * (kPKV / 8) / NT;  // 16-byte chunks per thread
    extern __shared__ __attribute__((aligned(16))) _Float16 smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = NG == 2 ? wave >> 2 : 0, wq = wave & 3;
    const int g = lane >> 5, j = lane & 31;
    const int M = (int)p.M, Mp = (int)p.Mp;
    const int qtiles = (M + kBQ - 1) / kBQ;
    const int pr = (int)blockIdx.x / (int)p.H, h = (int)blockIdx.x % (int)p.H;
    const int qa = pr, qb = qtiles - 1 - pr;
    auto tiles_for = [&](int qt) { return (min((qt + 1) * kBQ, M) - 1) / kPKV + 1; };
    const int Tl = qa == qb ? 0 : tiles_for(qa);
    const int Th = tiles_for(qb);

    const size_t head_elems = (size_t)M * D;
    const int hk = p.Hkv ? h / ((int)p.H / (int)p.Hkv) : h;
    const uint32_t cbytes = (uint32_t)((size_t)Mp * D * 2);
    auto kr = make_rsrc(p.Kf + (size_t)hk * Mp * D, cbytes);
    auto vr = make_rsrc(p.Vtf + (size_t)hk * Mp * D, cbytes);
    auto qr_ = make_rsrc(p.Q + (size_t)h * head_elems, (uint32_t)(head_elems * 2));

    // ---- K / V^T tiles: fetched 3 tiles ahead into registers, written to
    // the LDS ring 2 tiles ahead.  Keys past Mp read zeros: for K the offset
    // runs past the head's cache, for V^T (rows of Mp keys per dim) a chunk
    // past Mp would be the next dim's first keys, so its offset is made
    // out of range -- a masked key must not carry an inf or NaN into P V. ----
    // V^T chunk c of a tile (16 bytes: 8 keys of one dim row).  An 8-byte
    // LDS write pass serves 16 lanes on the 32 banks; at D = 64 (16 chunks per
    // 66-dword row) 16 chunks of one row would put chunks k and k + 8 on the
    // same banks, so a pass takes 8 chunks each of two adjacent rows (the
    // second row lands 2 banks over).  At D = 128 (8 chunks per row) one pass
    // already spans two rows.
    auto vchunk = [&](int c, int& row, int& ch) {
        constexpr int CPR = kPKV / 8;
        if constexpr (CPR == 16) {
            const int b = c >> 4, l = c & 15;
            row = 2 * (b >> 1) + (l >> 3);
            ch = 8 * (b & 1) + (l & 7);
        } else {
            row = c / CPR;
            ch = c % CPR;
        }
    };
    struct Raw { u4_t k[KCH], v[VCH]; };
    auto fetch = [&](int t, Raw& r) {
        const int k0 = t * kPKV;
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + NT * i;
            r.k[i] = ld_b128(kr, (uint32_t)((k0 + c / (D / 8)) * D + (c % (D / 8)) * 8) * 2u);
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            int vrow, vch;
            vchunk(tid + NT * i, vrow, vch);
            const int key = k0 + vch * 8;  // Mp is a multiple of 8: whole chunks in or out
            r.v[i] = ld_b128(vr, key < Mp ? (uint32_t)(vrow * Mp + key) * 2u : kOOB);
        }
    };
    auto kbuf = [&](int slot) { return smem + slot * TILE; };
    auto vbuf = [&](int slot) { return smem + slot * TILE + KT; };
    auto stage = [&](const Raw& r, int slot) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + NT * i;
            *reinterpret_cast<u4_t*>(kbuf(slot) + (c / (D / 8)) * KROW + (c % (D / 8)) * 8) = r.k[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            int vrow, vch;
            vchunk(tid + NT * i, vrow, vch);
            _Float16* dst = vbuf(slot) + vrow * VROW + vch * 8;
            if constexpr (VROW % 8 == 0) {
                *reinterpret_cast<u4_t*>(dst) = r.v[i];
            } else {  // rows 8-byte aligned only
                reinterpret_cast<u2_t*>(dst)[0] = u2_t{r.v[i].x, r.v[i].y};
                reinterpret_cast<u2_t*>(dst)[1] = u2_t{r.v[i].z, r.v[i].w};
            }
        }
    };

    // ---- this wave's units (key start 32 * unit index within the keys):
    // segment 1 = units 0..3 of tiles [0, Tl) (light queries for group 0,
    // heavy for group 1); segment 2 = tiles [Tl, Th) on the heavy queries, in
    // pairs (group 0 the first tile of a pair, group 1 the second, all four
    // units) and, when their count is odd, a last tile split two units per
    // group.  Each keeps the units whose first key is at or below the wave's
    // last query (n1: group 0's light units). ----
    const int qwL = qa * kBQ + wq * 32, qwH = qb * kBQ + wq * 32;
    const int n1 = grp == 0 ? (Tl > 0 ? min(UPT * Tl, (qwL + 31) / 32 + 1) : 0) : UPT * Tl;

    float c = p.scale * 1.4426950408889634f;  // log2 units
    const bool neg = c < 0.0f;
    if (neg) c = -c;

    h8_t qf[D / 16];
    auto load_q = [&](int qw, h8_t* dst) {
#pragma unroll
        for (int kk = 0; kk < D / 16; kk++) {
            const int my_q = qw + j;
            const uint32_t off = my_q < M ? ((uint32_t)my_q * D + kk * 16 + 8 * g) * 2u : kOOB;
            dst[kk] = __builtin_bit_cast(h8_t, ld_b128(qr_, off));
            if (neg) dst[kk] = -dst[kk];
        }
    };
    // group 0 starts on the light queries when it has any, else on the heavy ones
    bool light = grp == 0 && n1 > 0;
    int qw = light ? qwL : qwH;
    load_q(qw, qf);

    float m_run = -INFINITY;
    float l_run = 0.0f;  // this lane's half of the row sum of P
    f16v_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = f16v_t{};
    const h2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};

    auto store = [&](float inv) {
        const int my_q = qw + j;
        if (my_q >= M) return;
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int d0 = t * 32 + 8 * r4 + 4 * g;
                const f2_t a = {o[t][4 * r4] * inv, o[t][4 * r4 + 1] * inv};
                const f2_t b = {o[t][4 * r4 + 2] * inv, o[t][4 * r4 + 3] * inv};
                const size_t idx = p.o_token_major ? ((size_t)my_q * p.H + h) * D + d0
                                                   : (size_t)h * head_elems + (size_t)my_q * D + d0;
                *reinterpret_cast<u2_t*>(p.O + idx) =
                    u2_t{as_u32(__builtin_convertvector(a, h2_t)), as_u32(__builtin_convertvector(b, h2_t))};
            }
    };

    // ---- one unit: S^T of unit (slot, hh) is in s_in; the look-ahead unit's
    // S^T (ring slot nsl, unit hn) is computed into s_out beside the softmax;
    // MASK applies the causal / length mask to s_in first ----
    const int kbase = j * KROW + 8 * g, vbase = j * VROW + 4 * g;
    auto unit_core = [&](int slot, int hh, int key0, bool mask, f16v_t& s_in, int nsl, int hn, f16v_t& s_out) {
        if (mask) {
            const int my_q = qw + j;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = key0 + 8 * (r >> 2) + 4 * g + (r & 3);
                s_in[r] = (key <= my_q && key < M) ? s_in[r] : -INFINITY;
            }
        }
        // V^T fragments of this unit, K fragments of the look-ahead unit
        // (at D = 128 the second halves are read inside the chunk schedule,
        // once the registers of the first halves are free)
        u4_t va[2][DT];
        const _Float16* Vb = smem + slot * TILE + KT + hh * 32 + vbase;
        auto read_va = [&](int t2) {
#pragma unroll
            for (int tt = 0; tt < DT; tt++) {
                const _Float16* row = Vb + tt * 32 * VROW + t2 * 16;
                const u2_t lo = *reinterpret_cast<const u2_t*>(row);
                const u2_t hi = *reinterpret_cast<const u2_t*>(row + 8);
                va[t2][tt] = u4_t{lo.x, lo.y, hi.x, hi.y};
            }
        };
        h8_t kn_[D / 16];
        const _Float16* Kb = smem + nsl * TILE + hn * 32 * KROW + kbase;
        auto read_kn = [&](int kk0, int kk1) {
#pragma unroll
            for (int kk = kk0; kk < kk1; kk++) kn_[kk] = *reinterpret_cast<const h8_t*>(Kb + kk * 16);
        };
        read_va(0);
        if constexpr (D == 64) {
            read_va(1);
            read_kn(0, D / 16);
        } else {
            read_kn(0, 4);
        }
        // Row maximum: each lane's half (16 keys) decides whether the shared
        // reference point must move; only then are the two halves combined.
        float mx[4];  // a shallow tree of three-input maxima
#pragma unroll
        for (int q = 0; q < 4; q++) mx[q] = fmaxf(fmaxf(s_in[4 * q], s_in[4 * q + 1]), fmaxf(s_in[4 * q + 2], s_in[4 * q + 3]));
        const float hmax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
        const float m_cand = hmax * c;
        if (__any(m_cand > m_run + 8.0f)) {
            const float m_new = fmaxf(m_run, fmaxf(m_cand, __shfl_xor(m_cand, 32)));
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
#pragma unroll
            for (int tt = 0; tt < DT; tt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[tt][r] *= alpha;
            l_run *= alpha;
        }
        // --- fenced chunks: look-ahead S MFMAs and this unit's O MFMAs
        // interleaved with this unit's exponentials ---
        uint32_t pk[8];
        float e[16];
        auto exps = [&](int r0) {  // exp2 of accumulator rows r0 .. r0 + 3
#pragma unroll
            for (int r = r0; r < r0 + 4; r++)
                e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_in[r], c, -m_run));
        };
        auto cvts = [&](int r0) {  // P (fp16 pairs) of rows r0 .. r0 + 3
#pragma unroll
            for (int r = r0; r < r0 + 4; r += 2) {
                const h2_t pp = __builtin_convertvector((f2_t){e[r], e[r + 1]}, h2_t);
                pk[r >> 1] = as_u32(pp);
                l_run = __builtin_amdgcn_fdot2(pp, one2, l_run, false);  // row sum of the rounded P
            }
        };
        auto pv = [&](int t2, int tt) {
            const h8_t b = __builtin_bit_cast(h8_t, u4_t{pk[4 * t2], pk[4 * t2 + 1], pk[4 * t2 + 2], pk[4 * t2 + 3]});
            o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, va[t2][tt]), b, o[tt], 0, 0, 0);
        };
        auto smf = [&](int kk) {  // look-ahead S^T MFMA over d = 16 kk .. 16 kk + 15
            s_out = __builtin_amdgcn_mfma_f32_32x32x16_f16(kn_[kk], qf[kk], kk ? s_out : f16v_t{}, 0, 0, 0);
        };
        // raised wave priority for the interleaved block: the SIMD's other
        // wave (in its row-max / fragment-read phase) yields issue slots to it
        __builtin_amdgcn_s_setprio(1);
        // each exponential is converted one chunk after it is issued, and each
        // O MFMA follows the conversions it needs by a chunk where possible
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D == 64) {
            smf(0);
            exps(0);
            __builtin_amdgcn_sched_barrier(0);
            smf(1);
            exps(4);
            cvts(0);
            __builtin_amdgcn_sched_barrier(0);
            smf(2);
            exps(8);
            cvts(4);
            __builtin_amdgcn_sched_barrier(0);
            smf(3);
            pv(0, 0);
            exps(12);
            cvts(8);
            __builtin_amdgcn_sched_barrier(0);
            pv(0, 1);
            cvts(12);
            __builtin_amdgcn_sched_barrier(0);
            pv(1, 0);
            pv(1, 1);
        } else {  // D = 128: twice the MFMAs per unit against the same softmax
            smf(0);
            smf(1);
            exps(0);
            __builtin_amdgcn_sched_barrier(0);
            smf(2);
            smf(3);
            exps(4);
            cvts(0);
            read_kn(4, 8);
            __builtin_amdgcn_sched_barrier(0);
            smf(4);
            smf(5);
            exps(8);
            cvts(4);
            __builtin_amdgcn_sched_barrier(0);
            smf(6);
            smf(7);
            pv(0, 0);
            pv(0, 1);
            exps(12);
            cvts(8);
            read_va(1);
            __builtin_amdgcn_sched_barrier(0);
            pv(0, 2);
            pv(0, 3);
            cvts(12);
            __builtin_amdgcn_sched_barrier(0);
            pv(1, 0);
            pv(1, 1);
            pv(1, 2);
            pv(1, 3);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };
    auto scores_now = [&](int slot, int hh, f16v_t& s) {
        const _Float16* Kb = smem + slot * TILE + hh * 32 * KROW + kbase;
        h8_t ka[D / 16];
#pragma unroll
        for (int kk = 0; kk < D / 16; kk++) ka[kk] = *reinterpret_cast<const h8_t*>(Kb + kk * 16);
        s = f16v_t{};
#pragma unroll
        for (int kk = 0; kk < D / 16; kk++) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kk], qf[kk], s, 0, 0, 0);
    };
    auto switch_to_heavy = [&]() {  // light queries done: write them, take the heavy ones
        store(1.0f / (l_run + __shfl_xor(l_run, 32)));
        light = false;
        qw = qwH;
        load_q(qwH, qf);
        m_run = -INFINITY;
        l_run = 0.0f;
#pragma unroll
        for (int tt = 0; tt < DT; tt++) o[tt] = f16v_t{};
    };

    // ---- main loop.  Invariant at the start of a step at tile t: tiles t and
    // t + 1 are staged in ring slots t % 4, (t + 1) % 4 and visible, and `raw`
    // holds tile t + 2.  A single step (segment 1, or a last odd tile of
    // segment 2) stages t + 2, fetches t + 3 and takes tile t: group 0 the light
    // queries (then the heavy ones), group 1 the heavy ones, four units each;
    // on the last odd tile of segment 2 each group takes two units.  A double
    // step (segment 2) takes tiles t and t + 1: group 0 all units of tile t,
    // group 1 all units of tile t + 1 (heavy queries), and stages t + 2 and
    // t + 3, so a barrier serves eight units per wave instead of four.  Every
    // slot written held a tile finished before an earlier barrier.  The
    // look-ahead S MFMAs go into the next tile where that tile is already
    // visible: not across a double step's end, nor for group 1 into segment 2. ----
    int k = 0;          // light units done (group 0, segment 1)
    bool have = false;  // sA holds S^T of this wave's next unit
    f16v_t sA, sB;
    // units u0 .. u0 + nu - 1 of tile t whose first key is at or below the wave's heavy queries
    auto units_heavy = [&](int t, int u0, int nu) {
        int n = 0;
#pragma unroll
        for (int u = 0; u < UPT; u++) n += (u >= u0 && u < u0 + nu && t * kPKV + u * 32 <= qwH + 31) ? 1 : 0;
        return n;
    };
    const int Tdbl = Tl + ((Th - Tl) & ~1);  // double steps over [Tl, Tdbl); a single split step at Tdbl if odd
    // this wave's units in single-step tile t, and the first of them
    auto count_single = [&](int t) {
        if (t < Tl) return grp == 0 ? min(max(n1 - UPT * t, 0), UPT) : units_heavy(t, 0, UPT);
        return units_heavy(t, grp * (UPT / 2), UPT / 2);
    };
    auto first_single = [&](int t) { return t < Tl ? 0 : grp * (UPT / 2); };

    // cnt units of tile t (ring slot `slot`) from unit h0, S^T of the first in
    // sA when `have`; the last unit's look-ahead goes to (s_next, h_next) when next_ok
    auto run_tile = [&](int t, int slot, int cnt, int h0, bool next_ok, int s_next, int h_next) {
        if (cnt == 0) return;
        const int key_t = t * kPKV;
        const bool full = cnt == ((NG == 2 && t >= Tdbl && t >= Tl) ? UPT / 2 : UPT) && cnt >= 2;
        const bool unmasked = key_t + kPKV - 1 <= qw && key_t + kPKV <= M;
        if (full && unmasked) {
            // fast path: straight-line units, scores ping-ponging between sA and sB
            if (!have) scores_now(slot, h0, sA);
            const int sn = next_ok ? s_next : slot, hn = next_ok ? h_next : h0;
            if (UPT == 4 && cnt == 4) {
                unit_core(slot, h0, 0, false, sA, slot, h0 + 1, sB);
                unit_core(slot, h0 + 1, 0, false, sB, slot, h0 + 2, sA);
                unit_core(slot, h0 + 2, 0, false, sA, slot, h0 + 3, sB);
                unit_core(slot, h0 + 3, 0, false, sB, sn, hn, sA);
            } else {
                unit_core(slot, h0, 0, false, sA, slot, h0 + 1, sB);
                unit_core(slot, h0 + 1, 0, false, sB, sn, hn, sA);
            }
            have = next_ok;
        } else {
            // general path: up to four units, each with the mask where needed
#pragma unroll
            for (int u = 0; u < UPT; u++) {
                if (u < cnt) {
                    const int hh = h0 + u;
                    if (!have) scores_now(slot, hh, sA);
                    const bool last = u + 1 == cnt;
                    const int nsl = last ? (next_ok ? s_next : slot) : slot;
                    const int hn = last ? (next_ok ? h_next : hh) : hh + 1;
                    const int key0 = key_t + hh * 32;
                    unit_core(slot, hh, key0, key0 + 31 > qw || key0 + 31 >= M, sA, nsl, hn, sB);
                    sA = sB;
                    have = !last || next_ok;
                }
            }
        }
    };

    if constexpr (NG == 1) {
        // One group: the light tile's key tiles [0, Tl), then the heavy tile's
        // [0, Th), as one stream of Tl + Th steps through the ring (the first
        // Tl tiles are fetched twice).  Each wave switches to the heavy
        // queries after its last light unit and idles until step Tl.
        const int S = Tl + Th;
        auto tile_of = [&](int s) { return s < Tl ? s : s - Tl; };
        auto count_at = [&](int s) {
            return s < Tl ? min(max(n1 - UPT * s, 0), UPT) : units_heavy(s - Tl, 0, UPT);
        };
        Raw raw;
        fetch(tile_of(0), raw);
        stage(raw, 0);
        fetch(tile_of(1), raw);
        stage(raw, 1);
        fetch(tile_of(2), raw);
        __syncthreads();
        // step s: the units of tile_of(s); la: tile s + 1 is visible (look-ahead allowed)
        auto do_step = [&](int s, bool la) {
            const int cnt = count_at(s);
            const bool set_ends = light && s < Tl && k + cnt == n1;
            const bool next_ok = la && !set_ends && s + 1 < S && count_at(s + 1) > 0;
            run_tile(tile_of(s), s & 3, cnt, 0, next_ok, (s + 1) & 3, 0);
            if (s < Tl) k += cnt;
            if (set_ends) switch_to_heavy();
        };
        // Invariant at the start of an iteration at s: steps s and s + 1 are
        // staged and visible, `raw` holds s + 2.  Two steps per barrier: s + 2
        // is staged first, s + 3 after both steps (its slot held s - 1).
        for (int s = 0; s < S;) {
            const bool dbl = s + 1 < S;
            if (s + 2 < S) stage(raw, (s + 2) & 3);
            if (s + 3 < S) fetch(tile_of(s + 3), raw);
            do_step(s, true);
            if (dbl) {
                do_step(s + 1, false);
                if (s + 3 < S) stage(raw, (s + 3) & 3);
                if (s + 4 < S) fetch(tile_of(s + 4), raw);
            }
            __syncthreads();
            s += dbl ? 2 : 1;
        }
        const float l = l_run + __shfl_xor(l_run, 32);
        store(l > 0.0f ? 1.0f / l : 0.0f);
    } else {
        // ---- prologue ----
        Raw raw;
        fetch(0, raw);
        stage(raw, 0);
        fetch(1, raw);
        stage(raw, 1);
        fetch(2, raw);
        __syncthreads();

        int t = 0;
        while (t < Th) {
            const bool dbl = t >= Tl && t < Tdbl;
            if (t + 2 < Th) stage(raw, (t + 2) & 3);
            if (t + 3 < Th) fetch(t + 3, raw);  // double step: staged at its end
            int mt = t, cnt, h0 = 0, h_next = 0;
            bool next_ok = false, set_ends = false;
            if (!dbl) {
                cnt = count_single(t);
                h0 = first_single(t);
                // look-ahead of the tile's last unit: this wave's first unit of the
                // next step, when that step starts it at tile t + 1 (visible) with the
                // same queries
                set_ends = light && k + cnt == n1;
                if (!set_ends && t + 1 < Th) {
                    if (t + 1 < Tl || t + 1 >= Tdbl) {
                        next_ok = count_single(t + 1) > 0;
                        h_next = first_single(t + 1);
                    } else if (grp == 0) {  // next: a double step, whose first tile is group 0's
                        next_ok = units_heavy(t + 1, 0, UPT) > 0;
                    }
                }
            } else {
                mt = t + grp;  // this group's tile of the pair
                cnt = units_heavy(mt, 0, UPT);
            }
            run_tile(mt, mt & 3, cnt, h0, next_ok, (t + 1) & 3, h_next);
            if (!dbl) {
                if (t < Tl && grp == 0) k += cnt;
                if (set_ends) switch_to_heavy();
            } else {
                if (t + 3 < Th) stage(raw, (t + 3) & 3);
                if (t + 4 < Th) fetch(t + 4, raw);
            }
            __syncthreads();
            t += dbl ? 2 : 1;
        }

        // ---- merge group 0's partial state for the heavy queries into group 1's ----
        // One record of DT * 16 + 2 floats per lane (o, l, m), padded to a
        // multiple of 4 floats and written as 16-byte vectors: a lane stride
        // of 4 (mod 8) dwords puts the 16 lanes of a vector access on
        // distinct banks.
        constexpr int SW = (DT * 16 + 2 + 3) / 4 * 4 + ((((DT * 16 + 2 + 3) / 4) & 1) ? 0 : 4);
        float* X = reinterpret_cast<float*>(smem);
        static_assert(4 * 64 * SW * 4 <= NBUF * TILE * 2, "merge buffer fits the tile ring");
        float* x = X + (wq * 64 + lane) * SW;
        if (grp == 0) {
    #pragma unroll
            for (int t = 0; t < DT; t++)
    #pragma unroll
                for (int r = 0; r < 16; r += 4)
                    *reinterpret_cast<f4_t*>(x + t * 16 + r) = f4_t{o[t][r], o[t][r + 1], o[t][r + 2], o[t][r + 3]};
            *reinterpret_cast<f2_t*>(x + DT * 16) = f2_t{l_run, m_run};
        }
        __syncthreads();
        if (grp == 1) {
            const f2_t lm = *reinterpret_cast<const f2_t*>(x + DT * 16);
            const float ma = lm.y;
            const float m = fmaxf(ma, m_run);
            const float fa = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ma - m);
            const float fb = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
    #pragma unroll
            for (int t = 0; t < DT; t++)
    #pragma unroll
                for (int r = 0; r < 16; r += 4) {
                    const f4_t v = *reinterpret_cast<const f4_t*>(x + t * 16 + r);
                    o[t][r] = o[t][r] * fb + v.x * fa;
                    o[t][r + 1] = o[t][r + 1] * fb + v.y * fa;
                    o[t][r + 2] = o[t][r + 2] * fb + v.z * fa;
                    o[t][r + 3] = o[t][r + 3] * fb + v.w * fa;
                }
            const float lh = l_run * fb + lm.x * fa;
            const float l = lh + __shfl_xor(lh, 32);
            store(l > 0.0f ? 1.0f / l : 0.0f);
        }
    }
}
// LDS of the pipelined kernel: the 4-deep ring of K [key][D + 8] and V^T [D][key + 4] tiles
constexpr size_t pipe_lds(int D) { return 4 * (size_t)(pipe_keys(D) * (D + 8) + D * (pipe_keys(D) + kPVPad)) * 2; }

template <int D, int NG>
static hipError_t launch_pipe(const AttnParams& p, hipStream_t st) {
    const uint32_t qtiles = (p.M + kBQ - 1) / kBQ;  // a workgroup takes a light and a heavy query tile
    static size_t attr[kMaxDevices] = {};  // the tile ring needs more than the default 64 KB of LDS
    const hipError_t e = lds_limit_once((const void*)flash_attn_pipe_kernel<D, NG>, pipe_lds(D), attr);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((flash_attn_pipe_kernel<D, NG>), dim3(((qtiles + 1) / 2) * p.H), dim3(256 * NG), pipe_lds(D), st, p);
    return hipGetLastError();
}

hipError_t launch_flash_attn_q8_0(const AttnParams& p, hipStream_t st) {
    // the kernels read the dequantized fp16 cache (launch_kv_prep)
    if (p.Kf == nullptr || p.Vtf == nullptr || p.Mp < p.M || p.Mp % kBKV) return hipErrorInvalidValue;
    switch (p.D) {
        case 64: return launch_pipe<64, 2>(p, st);
        case 128: return launch_pipe<128, 1>(p, st);
        default: return hipErrorInvalidValue;
    }
}

uint32_t kv_padded_len(uint32_t M) { return (M + kBKV - 1) / kBKV * kBKV; }

hipError_t launch_kv_prep(const void* K, const void* V, bool from_q8, _Float16* Kf, _Float16* Vtf, uint32_t Hkv,
                          uint32_t M, uint32_t D, hipStream_t st, uint8_t* Kq, uint8_t* Vq) {
    const uint32_t Mp = kv_padded_len(M);
    dim3 grid(Mp / kBKV, Hkv);
    if (from_q8) Kq = Vq = nullptr;  // the blocks are the input
    switch (D * 2 + (from_q8 ? 1 : 0)) {
        case 128: hipLaunchKernelGGL((kv_prep_kernel<64, false>), grid, dim3(256), 0, st, K, V, Kf, Vtf, Kq, Vq, M, Mp); break;
        case 129: hipLaunchKernelGGL((kv_prep_kernel<64, true>), grid, dim3(256), 0, st, K, V, Kf, Vtf, Kq, Vq, M, Mp); break;
        case 256: hipLaunchKernelGGL((kv_prep_kernel<128, false>), grid, dim3(256), 0, st, K, V, Kf, Vtf, Kq, Vq, M, Mp); break;
        case 257: hipLaunchKernelGGL((kv_prep_kernel<128, true>), grid, dim3(256), 0, st, K, V, Kf, Vtf, Kq, Vq, M, Mp); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qr
