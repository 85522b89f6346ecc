// qr_dequant.hip -- [N, K] packed weights -> binary16 [N, K] on the GPU.
#include "qr_decode.h"
#include "qr_kernels.h"

namespace qr {

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
    decode_group<F>(raw, Dec::parity(n * col_bytes, g), o);
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
        case QUANT_VAR_RATE_AFFINE: hipLaunchKernelGGL(dequant_kernel<QUANT_VAR_RATE_AFFINE>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_EXL3: hipLaunchKernelGGL(dequant_kernel<QUANT_EXL3>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_Q8_0: hipLaunchKernelGGL(dequant_kernel<QUANT_Q8_0>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_PRISM_Q2_0: hipLaunchKernelGGL(dequant_kernel<QUANT_PRISM_Q2_0>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        case QUANT_MLX_4BIT_G64: hipLaunchKernelGGL(dequant_kernel<QUANT_MLX_4BIT_G64>, grid, dim3(256), 0, st, W, out, K, N, (uint32_t)col_bytes); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qr
