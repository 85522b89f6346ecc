// qr_attention.hip -- Q8_0 KV-cache quantization and causal flash attention
// over the Q8_0 cache on gfx950.
//
// Replaces quantize_kv_to_q8_0 (unified_kernels.metal:118-145) and
// flash_attn_mma_64x64_q8_0_impl<D> (brick4_attn_kernels.metal:572-881).
//
// Attention design (one workgroup = 4 wave64s = 128 queries of one head):
//  * Each wave owns 32 queries and computes S^T = K . Q^T with
//    v_mfma_f32_32x32x16_f16, so a lane owns ONE query column: the softmax
//    row statistics are lane-local over its 16 accumulator rows plus one
//    exchange with the partner lane (l ^ 32) -- no 32-lane reduction trees.
//  * K/V tiles of 64 keys are dequantized once per workgroup from Q8_0 into
//    LDS (K as [key][d], V transposed as [d][key]); the binary16 value is the
//    exact product q * d rounded once, as the reference's dequantizer
//    (brick4_attn_bench.mm:57-65).
//  * P stays in registers: the S^T accumulator of a lane already holds the
//    8 keys that lane must supply as the B operand of O^T = V^T . P^T, given
//    the matching key order in the V^T A-operand reads (two ds_read_b64).
//  * fp32 running max / sum / output accumulators (the reference keeps
//    S, P and O in half); the output is rounded to fp16 once.
#include "qr_device.h"
#include "qr_kernels.h"

namespace qr {

// --------------------------------------------------------------------------
// Q8_0 quantization: per 32 values amax in fp32, d = amax / 127 (IEEE
// division), stored as half(d); codes q = round(x * (1/d)) (half away from
// zero) with the UNROUNDED d, clamped to [-128, 127] (unified_kernels.metal:
// 118-145).  One thread per block.
// --------------------------------------------------------------------------
__global__ void __launch_bounds__(256) quantize_q8_0_kernel(const _Float16* src, uint8_t* dst, size_t nblocks) {
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    const u4_t* s = reinterpret_cast<const u4_t*>(src + b * 32);
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        u4_t v = s[i];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        x[2 * i] = h2f(w[i] & 0xffffu);
        x[2 * i + 1] = h2f(w[i] >> 16);
        amax = fmaxf(amax, fabsf(x[2 * i]));
        amax = fmaxf(amax, fabsf(x[2 * i + 1]));
    }
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint16_t* o16 = reinterpret_cast<uint16_t*>(dst + b * 34);  // 34-byte blocks are 2-byte aligned
    o16[0] = (uint16_t)f2h_bits(d);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        int q0 = (int)__builtin_roundf(x[2 * i] * id);
        int q1 = (int)__builtin_roundf(x[2 * i + 1] * id);
        q0 = q0 < -128 ? -128 : (q0 > 127 ? 127 : q0);
        q1 = q1 < -128 ? -128 : (q1 > 127 ? 127 : q1);
        o16[1 + i] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
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
constexpr int kBQ = 128;      // queries per workgroup
constexpr int kBKV = 64;      // keys per tile

// Dequantize one Q8_0 block (34 bytes at byte offset o of the rsrc) into 16
// half2 words: w[p] = {q[2p] * d, q[2p+1] * d}, each rounded once.
__device__ __forceinline__ void q8_block_to_h2(__amdgpu_buffer_rsrc_t r, uint32_t o, uint32_t out[16]) {
    const uint32_t a = o & ~3u;
    uint32_t raw[10];
#pragma unroll
    for (int i = 0; i < 9; i++) raw[i] = ld_b32(r, a + 4u * i);
    raw[9] = 0;
    const bool par = (o & 2u) != 0;
    const uint32_t d16 = par ? (raw[0] >> 16) : (raw[0] & 0xffffu);
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = par ? raw[i + 1] : __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2);
    const h2_t d = as_h2(d16 | (d16 << 16));
    const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t u = q[i] ^ 0x80808080u;  // two's complement byte -> q + 128
        out[2 * i] = as_u32((as_h2(nib_pair_lo(u)) - off) * d);
        out[2 * i + 1] = as_u32((as_h2(nib_pair_hi(u)) - off) * d);
    }
}

template <int D>
__global__ void __launch_bounds__(256) flash_attn_q8_0_kernel(AttnParams p) {
    constexpr int NB = D / 32;                 // Q8_0 blocks per token row
    constexpr int KROW = D + 8;                // LDS row (halfs) of K tile [key][d]
    constexpr int VROW = kBKV + 8;             // LDS row (halfs) of V^T tile [d][key]
    constexpr int DT = D / 32;                 // 32-row output tiles along d
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kBKV * KROW];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, j = lane & 31;
    const uint32_t M = p.M;
    const int qtiles = (int)((M + kBQ - 1) / kBQ);
    const int qt = qtiles - 1 - (int)blockIdx.x;   // heaviest (latest) tiles first
    const int h = blockIdx.y;
    const int q0 = qt * kBQ;
    const int qw = q0 + wave * 32;                 // this wave's first query
    const int my_q = qw + j;                       // this lane's query

    const size_t head_elems = (size_t)M * D;
    const _Float16* Qh = p.Q + (size_t)h * head_elems;
    const uint32_t kv_bytes = (uint32_t)(head_elems / 32 * 34);
    auto kr = make_rsrc(p.Kq + (size_t)h * (head_elems / 32) * 34, kv_bytes);
    auto vr = make_rsrc(p.Vq + (size_t)h * (head_elems / 32) * 34, kv_bytes);

    // Q^T fragments (B operand): lane holds Q[my_q][kk*16 + 8g .. +7].
    h8_t qf[D / 16];
    {
        auto qr_ = make_rsrc(Qh, (uint32_t)(head_elems * 2));
#pragma unroll
        for (int kk = 0; kk < D / 16; kk++) {
            uint32_t off = my_q < (int)M ? ((uint32_t)my_q * D + kk * 16 + 8 * g) * 2u : kOOB;
            u4_t v = ld_b128(qr_, off);
            qf[kk] = __builtin_bit_cast(h8_t, v);
        }
    }

    const float sl2 = p.scale * 1.4426950408889634f;  // scores in log2 units
    float m_run = -INFINITY, l_run = 0.0f;
    f16v_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = f16v_t{};

    const int q_last = min(q0 + kBQ, (int)M) - 1;
    const int ntiles = q_last / kBKV + 1;

    for (int kt = 0; kt < ntiles; kt++) {
        const int k0 = kt * kBKV;
        __syncthreads();  // previous tile fully consumed
        // ---- dequantize K and V tiles into LDS: 2 * 64 * NB blocks ----
        for (int bi = tid; bi < 2 * kBKV * NB; bi += 256) {
            const bool isv = bi >= kBKV * NB;
            const int b = isv ? bi - kBKV * NB : bi;
            const int key = b % kBKV, db = b / kBKV;   // adjacent lanes: adjacent keys
            const int gk = k0 + key;
            uint32_t off = gk < (int)M ? (uint32_t)(gk * NB + db) * 34u : kOOB;
            uint32_t w[16];
            q8_block_to_h2(isv ? vr : kr, off, w);
            if (!isv) {
                u4_t* dst = reinterpret_cast<u4_t*>(Ks + key * KROW + db * 32);
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = u4_t{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
            } else {
                uint16_t* vt = reinterpret_cast<uint16_t*>(Vt);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    vt[(db * 32 + 2 * i) * VROW + key] = (uint16_t)(w[i] & 0xffffu);
                    vt[(db * 32 + 2 * i + 1) * VROW + key] = (uint16_t)(w[i] >> 16);
                }
            }
        }
        __syncthreads();
        if (k0 > qw + 31) continue;  // whole tile above this wave's diagonal

        // ---- S^T = K . Q^T : two 32-key tiles ----
        f16v_t s[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            s[ks] = f16v_t{};
#pragma unroll
            for (int kk = 0; kk < D / 16; kk++) {
                h8_t a = *reinterpret_cast<const h8_t*>(Ks + (ks * 32 + j) * KROW + kk * 16 + 8 * g);
                s[ks] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], s[ks], 0, 0, 0);
            }
        }
        // ---- mask, scale, running max ----
        float tmax = -INFINITY;
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = k0 + ks * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                float v = s[ks][r] * sl2;
                v = (key <= my_q && key < (int)M) ? v : -INFINITY;
                s[ks][r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // exp2(-inf) = 0 on the first tile
        m_run = m_new;
        float lsum = 0.0f;
        uint32_t pk[2][8];  // P as half2 words in accumulator order
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                float e0 = __builtin_amdgcn_exp2f(s[ks][r] - m_new);
                float e1 = __builtin_amdgcn_exp2f(s[ks][r + 1] - m_new);
                lsum += e0 + e1;
                pk[ks][r >> 1] = pack_h2(f2h_bits(e0), f2h_bits(e1));
            }
        l_run = l_run * alpha + lsum;
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[t][r] *= alpha;

        // ---- O^T += V^T . P^T : 4 k16 steps over the 64 keys ----
        // step (ks, t2): B operand = P rows r = 8*t2 .. 8*t2+7 of tile ks, i.e. keys
        // 32ks + 16t2 + 4g + {0..3} and 32ks + 16t2 + 8 + 4g + {0..3}.
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                u4_t bw = {pk[ks][4 * t2], pk[ks][4 * t2 + 1], pk[ks][4 * t2 + 2], pk[ks][4 * t2 + 3]};
                h8_t b = __builtin_bit_cast(h8_t, bw);
                const int kb0 = ks * 32 + t2 * 16 + 4 * g;
#pragma unroll
                for (int t = 0; t < DT; t++) {
                    const _Float16* row = Vt + (t * 32 + j) * VROW;
                    u2_t lo = *reinterpret_cast<const u2_t*>(row + kb0);
                    u2_t hi = *reinterpret_cast<const u2_t*>(row + kb0 + 8);
                    u4_t aw = {lo.x, lo.y, hi.x, hi.y};
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, aw), b, o[t], 0, 0, 0);
                }
            }
    }

    // ---- normalize and store ----
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < (int)M) {
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int d0 = t * 32 + 8 * r4 + 4 * g;
                uint32_t w0 = pack_h2(f2h_bits(o[t][4 * r4] * inv), f2h_bits(o[t][4 * r4 + 1] * inv));
                uint32_t w1 = pack_h2(f2h_bits(o[t][4 * r4 + 2] * inv), f2h_bits(o[t][4 * r4 + 3] * inv));
                size_t idx = p.o_token_major ? ((size_t)my_q * p.H + h) * D + d0 : (size_t)h * head_elems + (size_t)my_q * D + d0;
                *reinterpret_cast<u2_t*>(p.O + idx) = u2_t{w0, w1};
            }
    }
}

hipError_t launch_flash_attn_q8_0(const AttnParams& p, hipStream_t st) {
    dim3 grid((p.M + kBQ - 1) / kBQ, p.H);
    switch (p.D) {
        case 64: hipLaunchKernelGGL(flash_attn_q8_0_kernel<64>, grid, dim3(256), 0, st, p); break;
        case 128: hipLaunchKernelGGL(flash_attn_q8_0_kernel<128>, grid, dim3(256), 0, st, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qr
