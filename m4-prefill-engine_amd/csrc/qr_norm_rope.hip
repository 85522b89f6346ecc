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

// One thread per (row, 8 consecutive pairs).  Angles are formed in double
// (pos * theta^(-2i/D), reduced modulo 2 pi) so long positions keep their
// precision; sin/cos of the reduced angle in fp32.
__global__ void __launch_bounds__(256) rope_kernel(_Float16* T, uint32_t rows, uint32_t M, uint32_t D, float theta,
                                                   uint32_t offset, int traditional) {
    const uint32_t half = D / 2, per_row = half / 8;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (size_t)rows * per_row) return;
    const size_t row = t / per_row;
    const uint32_t i0 = (uint32_t)(t % per_row) * 8;  // first pair index of this thread
    const double pos = (double)(offset + (uint32_t)(row % M));
    _Float16* x = T + row * D;
    float a[8], b[8];
    if (traditional) {  // pairs (2i, 2i + 1): 16 consecutive elements
        const h8_t u = *reinterpret_cast<const h8_t*>(x + 2 * i0);
        const h8_t v = *reinterpret_cast<const h8_t*>(x + 2 * i0 + 8);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            a[k] = (float)u[2 * k]; b[k] = (float)u[2 * k + 1];
            a[k + 4] = (float)v[2 * k]; b[k + 4] = (float)v[2 * k + 1];
        }
    } else {            // pairs (i, i + D/2)
        const h8_t u = *reinterpret_cast<const h8_t*>(x + i0);
        const h8_t v = *reinterpret_cast<const h8_t*>(x + i0 + half);
#pragma unroll
        for (int k = 0; k < 8; k++) { a[k] = (float)u[k]; b[k] = (float)v[k]; }
    }
    // inverse frequency of pair i0, then successive ratios theta^(-2/D)
    const double l2t = log2((double)theta);
    const double ratio = exp2(-2.0 / (double)D * l2t);
    double f = exp2(-2.0 * (double)i0 / (double)D * l2t);
    const double two_pi = 6.283185307179586476925286766559, inv_two_pi = 0.15915494309189533576888376337251;
    float ra[8], rb[8];
#pragma unroll
    for (int k = 0; k < 8; k++, f *= ratio) {
        const double ang = pos * f;
        const float red = (float)__builtin_fma(-two_pi, rint(ang * inv_two_pi), ang);
        const float sn = sinf(red), cs = cosf(red);
        ra[k] = a[k] * cs - b[k] * sn;
        rb[k] = a[k] * sn + b[k] * cs;
    }
    if (traditional) {
        h8_t u, v;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            u[2 * k] = (_Float16)ra[k]; u[2 * k + 1] = (_Float16)rb[k];
            v[2 * k] = (_Float16)ra[k + 4]; v[2 * k + 1] = (_Float16)rb[k + 4];
        }
        *reinterpret_cast<h8_t*>(x + 2 * i0) = u;
        *reinterpret_cast<h8_t*>(x + 2 * i0 + 8) = v;
    } else {
        h8_t u, v;
#pragma unroll
        for (int k = 0; k < 8; k++) { u[k] = (_Float16)ra[k]; v[k] = (_Float16)rb[k]; }
        *reinterpret_cast<h8_t*>(x + i0) = u;
        *reinterpret_cast<h8_t*>(x + i0 + half) = v;
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
    const size_t threads = (size_t)H * M * (D / 16);
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, T, H * M, M, D, theta,
                       offset, traditional);
    return hipGetLastError();
}

}  // namespace qr
