// qr_norm_rope.hip -- RMSNorm and rotary position embedding of the MLX block
// (src/engine/model.py:17-48 RMSNorm, :112-116 / :215-226 nn.RoPE), the two
// row-wise ops the router layer gains when it runs a full Llama/Gemma block.
// Both are HBM-bound elementwise passes: 16-byte loads and stores, fp32 math.
#include "qr_device.h"
#include "qr_kernels.h"

namespace qr {

// One wave per row; each lane owns 8-element chunks lane, lane + 64, ...
// Rows of up to 64 * 8 * CPL elements stay in registers between the sum of
// squares and the scaling (one HBM read); CPL = 0 streams the row twice.
template <int CPL>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const _Float16* X, const _Float16* w, _Float16* Y, uint32_t M,
                                                      uint32_t D, float eps, int gemma) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const _Float16* x = X + (size_t)row * D;
    const uint32_t chunks = D / 8;
    auto scale_store = [&](uint32_t c, const h8_t& v, float r) {
        const h8_t wv = *reinterpret_cast<const h8_t*>(w + 8 * c);
        h8_t o;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const _Float16 nv = (_Float16)((float)v[i] * r);                      // fp16(x r)
            const _Float16 ww = gemma ? (_Float16)(1.0f + (float)wv[i]) : wv[i];   // fp16(1 + w)
            o[i] = (_Float16)((float)nv * (float)ww);  // exact product, one rounding
        }
        *reinterpret_cast<h8_t*>(Y + (size_t)row * D + 8 * c) = o;
    };
    float ss = 0.0f;
    h8_t keep[CPL > 0 ? CPL : 1];
    if constexpr (CPL > 0) {
#pragma unroll
        for (int k = 0; k < CPL; k++) {
            const uint32_t c = lane + 64 * k;
            keep[k] = c < chunks ? *reinterpret_cast<const h8_t*>(x + 8 * c) : h8_t{};
        }
#pragma unroll
        for (int k = 0; k < CPL; k++)
#pragma unroll
            for (int i = 0; i < 8; i++) ss = __builtin_fmaf((float)keep[k][i], (float)keep[k][i], ss);
    } else {
        for (uint32_t c = lane; c < chunks; c += 64) {
            const h8_t v = *reinterpret_cast<const h8_t*>(x + 8 * c);
#pragma unroll
            for (int i = 0; i < 8; i++) ss = __builtin_fmaf((float)v[i], (float)v[i], ss);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float r = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    if constexpr (CPL > 0) {
#pragma unroll
        for (int k = 0; k < CPL; k++) {
            const uint32_t c = lane + 64 * k;
            if (c < chunks) scale_store(c, keep[k], r);
        }
    } else {
        for (uint32_t c = lane; c < chunks; c += 64) scale_store(c, *reinterpret_cast<const h8_t*>(x + 8 * c), r);
    }
}

// One thread per (position, 8 consecutive pairs, group of kRopeHeads heads):
// the angles depend only on the position and the pair, so they are formed
// once and applied to every head of the group.  Angles are formed in double
// (pos * theta^(-2i/D), reduced modulo 2 pi) so long positions keep their
// precision; sin/cos of the reduced angle in fp32.  T is [H, M, D].
constexpr uint32_t kRopeHeads = 4;

__global__ void __launch_bounds__(128) rope_kernel(_Float16* T, uint32_t H, uint32_t M, uint32_t D, float theta,
                                                   uint32_t offset, int traditional) {
    const uint32_t half = D / 2, per_row = half / 8;
    const size_t t = (size_t)blockIdx.x * 128 + threadIdx.x;
    if (t >= (size_t)M * per_row) return;
    const uint32_t m = (uint32_t)(t / per_row);
    const uint32_t i0 = (uint32_t)(t % per_row) * 8;  // first pair index of this thread
    const uint32_t h0 = blockIdx.y * kRopeHeads;
    const double pos = (double)(offset + m);
    // inverse frequency of pair i0, then successive ratios theta^(-2/D)
    const double l2t = log2((double)theta);
    const double ratio = exp2(-2.0 / (double)D * l2t);
    double f = exp2(-2.0 * (double)i0 / (double)D * l2t);
    const double two_pi = 6.283185307179586476925286766559, inv_two_pi = 0.15915494309189533576888376337251;
    float sn[8], cs[8];
#pragma unroll
    for (int k = 0; k < 8; k++, f *= ratio) {
        const double ang = pos * f;
        const float red = (float)__builtin_fma(-two_pi, rint(ang * inv_two_pi), ang);
        sn[k] = sinf(red);
        cs[k] = cosf(red);
    }
    // element offsets of the thread's two 8-element runs within a row
    const uint32_t o0 = traditional ? 2 * i0 : i0, o1 = traditional ? 2 * i0 + 8 : i0 + half;
    h8_t u[kRopeHeads], v[kRopeHeads];
#pragma unroll
    for (uint32_t j = 0; j < kRopeHeads; j++) {  // all loads first
        if (h0 + j < H) {
            const _Float16* x = T + ((size_t)(h0 + j) * M + m) * D;
            u[j] = *reinterpret_cast<const h8_t*>(x + o0);
            v[j] = *reinterpret_cast<const h8_t*>(x + o1);
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kRopeHeads; j++) {
        if (h0 + j >= H) break;
        float a[8], b[8];
        if (traditional) {  // pairs (2i, 2i + 1): 16 consecutive elements
#pragma unroll
            for (int k = 0; k < 4; k++) {
                a[k] = (float)u[j][2 * k]; b[k] = (float)u[j][2 * k + 1];
                a[k + 4] = (float)v[j][2 * k]; b[k + 4] = (float)v[j][2 * k + 1];
            }
        } else {            // pairs (i, i + D/2)
#pragma unroll
            for (int k = 0; k < 8; k++) { a[k] = (float)u[j][k]; b[k] = (float)v[j][k]; }
        }
        float ra[8], rb[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            ra[k] = a[k] * cs[k] - b[k] * sn[k];
            rb[k] = a[k] * sn[k] + b[k] * cs[k];
        }
        h8_t uo, vo;
        if (traditional) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uo[2 * k] = (_Float16)ra[k]; uo[2 * k + 1] = (_Float16)rb[k];
                vo[2 * k] = (_Float16)ra[k + 4]; vo[2 * k + 1] = (_Float16)rb[k + 4];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) { uo[k] = (_Float16)ra[k]; vo[k] = (_Float16)rb[k]; }
        }
        _Float16* x = T + ((size_t)(h0 + j) * M + m) * D;
        *reinterpret_cast<h8_t*>(x + o0) = uo;
        *reinterpret_cast<h8_t*>(x + o1) = vo;
    }
}

hipError_t launch_rmsnorm(const _Float16* X, const _Float16* w, _Float16* Y, uint32_t M, uint32_t D, float eps,
                          int norm_type, hipStream_t st) {
    if (D % 8 || (norm_type != 1 && norm_type != 2)) return hipErrorInvalidValue;
    const dim3 grid((M + 3) / 4);
    if (D <= 64 * 8 * 4)
        hipLaunchKernelGGL(rmsnorm_kernel<4>, grid, dim3(256), 0, st, X, w, Y, M, D, eps, norm_type == 2);
    else if (D <= 64 * 8 * 16)
        hipLaunchKernelGGL(rmsnorm_kernel<16>, grid, dim3(256), 0, st, X, w, Y, M, D, eps, norm_type == 2);
    else
        hipLaunchKernelGGL(rmsnorm_kernel<0>, grid, dim3(256), 0, st, X, w, Y, M, D, eps, norm_type == 2);
    return hipGetLastError();
}

hipError_t launch_rope(_Float16* T, uint32_t H, uint32_t M, uint32_t D, float theta, uint32_t offset,
                       int traditional, hipStream_t st) {
    if (D % 16) return hipErrorInvalidValue;
    if (H == 0 || M == 0) return hipSuccess;
    const size_t threads = (size_t)M * (D / 16);
    const dim3 grid((unsigned)((threads + 127) / 128), (H + kRopeHeads - 1) / kRopeHeads);
    hipLaunchKernelGGL(rope_kernel, grid, dim3(128), 0, st, T, H, M, D, theta, offset, traditional);
    return hipGetLastError();
}

}  // namespace qr
