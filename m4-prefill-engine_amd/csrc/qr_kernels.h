// qr_kernels.h -- host-visible launch interface of the router kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qr {

struct GemmParams {
    int format;
    const _Float16* X;    // [M, K] fp16, 16-byte aligned
    const uint8_t* W;     // [N, K] packed blocks, 16-byte aligned
    const uint8_t* W2;    // second weight matrix (SwiGLU up projection) or null
    _Float16* Y;          // output
    const _Float16* R;    // optional residual [M, N] added before rounding, or null
    uint32_t M, N, K;
    uint32_t head_D;      // 0: Y is [M, N]; else direct-head [N / head_D, M, head_D]
    size_t col_bytes;     // bytes of one weight column
    // K split across workgroups (tiled kernel): 0/1 = none.  `ws` holds
    // gemm_workspace_floats() floats of fp32 partials [split][plane][M][N];
    // launch_gemm follows the projection with the reduction kernel.
    uint32_t ksplit;
    float* ws;
    uint32_t group_m;     // row-tiles per XCD tile group (0: kernel default)
    // Grouped launch: up to two more projections of the same X (same K,
    // format, head_D; no residual, no SwiGLU, no K split) in the same grid,
    // group g >= 1 writing Yx[g - 1] [M, Nx[g - 1]] from Wx[g - 1].
    uint32_t ngroups;     // 0 or 1: a single projection
    const uint8_t* Wx[2];
    _Float16* Yx[2];
    uint32_t Nx[2];
};

hipError_t launch_gemm(const GemmParams& p, hipStream_t st);
uint32_t gemm_group_m(const GemmParams& p);
uint32_t gemm_pick_ksplit(const GemmParams& p);
// Whether launch_gemm can run p's groups (ngroups >= 2) as one grid.
bool gemm_grouped_ok(const GemmParams& p);
size_t gemm_workspace_floats(const GemmParams& p, uint32_t ksplit);
// Sums split-K partials ws [ks][dual ? 2 : 1][M][N] in split order and writes
// the projection epilogue (SwiGLU when dual, + R, fp16, head-major when
// head_D) -- the second kernel of every split-K projection.
hipError_t launch_splitk_reduce(const float* ws, uint32_t ks, uint32_t M, uint32_t N, bool dual, const _Float16* R,
                                _Float16* Y, uint32_t head_D, hipStream_t st);

// Small-M weight-streaming projection (M <= 64, no SwiGLU).  `ws` holds
// skinny_workspace_floats() floats of split-K partials [split][M][N], summed
// by launch_splitk_reduce.  Calls that share ws must be ordered on one stream.
bool skinny_supported(const GemmParams& p);
size_t skinny_workspace_floats(uint32_t M, uint32_t N, uint32_t K);
hipError_t launch_gemm_skinny(const GemmParams& p, float* ws, hipStream_t st);
hipError_t launch_dequant(int format, const uint8_t* W, _Float16* out, uint32_t K, uint32_t N, size_t col_bytes,
                          hipStream_t st);

// Q8_0 quantization of `num_blocks` groups of 32 fp16 values.
hipError_t launch_quantize_q8_0(const _Float16* src, uint8_t* dst, size_t num_blocks, hipStream_t st);

struct AttnParams {
    const _Float16* Q;    // [H, M, D]
    _Float16* O;          // [H, M, D] or token-major [M, H * D]
    uint32_t H, M, D;
    float scale;
    int o_token_major;
    uint32_t Hkv;         // KV heads (grouped-query: query head h reads KV head h / (H / Hkv)); 0 = H
    // The dequantized fp16 cache of the Q8_0 K / V (launch_kv_prep):
    // Kf [Hkv, Mp, D], Vtf [Hkv, D, Mp], Mp = kv_padded_len(M).
    const _Float16* Kf;
    const _Float16* Vtf;
    uint32_t Mp;
};
hipError_t launch_flash_attn_q8_0(const AttnParams& p, hipStream_t st);
uint32_t kv_padded_len(uint32_t M);
// K / V ([Hkv, M, D] Q8_0 blocks when from_q8, else fp16) -> the dequantized
// fp16 cache of the attention kernel (Q8_0 values half(q * half(d)), computed
// from fp16 inputs by quantizing and dequantizing in registers).
// From fp16 K / V, the Q8_0 blocks are also written to Kq / Vq when non-null
// (the layer's Q8_0 KV cache, [Hkv, M, D] blocks of 32 d).
hipError_t launch_kv_prep(const void* K, const void* V, bool from_q8, _Float16* Kf, _Float16* Vtf, uint32_t Hkv,
                          uint32_t M, uint32_t D, hipStream_t st, uint8_t* Kq = nullptr, uint8_t* Vq = nullptr);

// RMSNorm over rows of X [M, D] (D % 8 == 0): y = fp16(fp16(x r) w), r =
// 1 / sqrt(mean(x^2) + eps); norm_type 2 uses fp16(1 + w) in place of w.
hipError_t launch_rmsnorm(const _Float16* X, const _Float16* w, _Float16* Y, uint32_t M, uint32_t D, float eps,
                          int norm_type, hipStream_t st);
// Rotary position embedding in place on T [H, M, D] (D % 16 == 0), positions
// offset + m, frequencies theta^(-2i/D); pairs (i, i + D/2), or (2i, 2i + 1)
// when traditional.
hipError_t launch_rope(_Float16* T, uint32_t H, uint32_t M, uint32_t D, float theta, uint32_t offset,
                       int traditional, hipStream_t st);

}  // namespace qr
