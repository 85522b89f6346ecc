// qr_probe.hip -- on-device roofline probes: the HBM bandwidth and matrix
// (MFMA) throughput this MI355X actually reaches, measured in the same run as
// the kernels they bound.
//
// Replaces the reference's hardware-ceiling probes probe_memory_bandwidth and
// probe_fma_roofline (quant_router_kernels.metal:71-104), timed by its bench
// (bench_universal_router.mm:645-717).  The reference probes the vector-ALU
// fp16 FMA rate and quotes a fixed matrix peak; here the matrix pipe itself
// is probed (v_mfma_f32_32x32x16_f16, the instruction every projection and
// attention kernel issues), together with the shader clock it ran at.
#include <hip/hip_runtime.h>

#include <cstdio>

#include "../../include/m4_mlx_bridge.h"
#include "qr_device.h"

namespace qr {

// Read-only stream: each thread sums 16-byte chunks (grid-stride), one word
// per thread written so the loads cannot be elided.  Bytes moved = the buffer.
__global__ void __launch_bounds__(256) probe_read_kernel(const u4_t* __restrict__ src, size_t n16,
                                                         uint32_t* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * 256;
    uint32_t acc = 0;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u4_t a = __builtin_nontemporal_load(src + i);
        const u4_t b = __builtin_nontemporal_load(src + i + stride);
        const u4_t c = __builtin_nontemporal_load(src + i + 2 * stride);
        const u4_t d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const u4_t a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

// The reference's bandwidth probe: dst = src + 1 on float4 (read + write).
__global__ void __launch_bounds__(256) probe_copy_kernel(const f4_t* __restrict__ src, f4_t* __restrict__ dst,
                                                         size_t n16) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i] + f4_t{1.0f, 1.0f, 1.0f, 1.0f};
}

// Matrix pipe: each wave runs kChains independent accumulator chains of
// v_mfma_f32_32x32x16_f16 (32 * 32 * 16 * 2 flop each), enough to cover the
// instruction's latency, for `iters` rounds.  Thread 0 of every workgroup
// records the shader-clock and constant 100 MHz counters around the loop, so
// the host can report the clock the matrix pipe ran at.
// RND = false: the same low-entropy operands every round (near 1.0 and powers
// of two); RND = true: every lane cycles through four random fp16 A and four
// B fragments from `tab` (values in [-1, 1)).  The matrix pipe's power, and
// with it the clock the part holds, depends on how many operand bits toggle,
// so the random form is the ceiling real activations and weights can reach.
constexpr int kChains = 4;
template <bool RND>
__global__ void __launch_bounds__(256) probe_mfma_kernel(float* __restrict__ out, uint32_t iters,
                                                         unsigned long long* __restrict__ clocks,
                                                         const h8_t* __restrict__ tab) {
    const int lane = threadIdx.x & 63;
    h8_t a[4], b[4];
    if constexpr (RND) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = tab[threadIdx.x * 8 + i];
            b[i] = tab[threadIdx.x * 8 + 4 + i];
        }
    } else {
        const _Float16 v = (_Float16)(1.0f + 0.001f * (float)(lane & 7));
        a[0] = h8_t{v, v, v, v, v, v, v, v};
        b[0] = h8_t{(_Float16)0.5f, (_Float16)0.25f, (_Float16)0.125f, (_Float16)0.5f,
                    (_Float16)0.25f, (_Float16)0.125f, (_Float16)0.5f, (_Float16)0.25f};
#pragma unroll
        for (int i = 1; i < 4; i++) {
            a[i] = a[0];
            b[i] = b[0];
        }
    }
    f16v_t acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; c++) acc[c] = f16v_t{};
    const unsigned long long c0 = __builtin_readcyclecounter();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; it += 4) {  // iters is a multiple of 4
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int c = 0; c < kChains; c++)
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(u + c) & 3], b[(3 * u + c) & 3], acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[c][r];
    const unsigned long long c1 = __builtin_readcyclecounter();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[2 * blockIdx.x] = c1 - c0;
        clocks[2 * blockIdx.x + 1] = r1 - r0;
    }
}

}  // namespace qr

namespace {

struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    Events() {
        (void)hipEventCreate(&a);
        (void)hipEventCreate(&b);
    }
    ~Events() {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
};

}  // namespace

extern "C" {

int m4_probe_hbm_bandwidth(size_t bytes, int reps, double* read_gbs, double* copy_gbs) {
    if (!read_gbs || !copy_gbs) return -2;
    if (bytes < (1u << 20) || reps < 1) return -4;
    bytes &= ~(size_t)15;
    const size_t n16 = bytes / 16;
    void *src = nullptr, *dst = nullptr, *sink = nullptr;
    const int blocks = 256 * 8;
    hipError_t e = hipMalloc(&src, bytes);
    if (e == hipSuccess) e = hipMalloc(&dst, bytes);
    if (e == hipSuccess) e = hipMalloc(&sink, (size_t)blocks * 256 * 4);
    if (e == hipSuccess) e = hipMemset(src, 1, bytes);
    Events ev;
    float best_r = 1e30f, best_c = 1e30f;
    // Alternate the two kernels: each read of the > 256 MB buffer evicts the
    // other's working set from the 256 MB Infinity Cache.
    for (int r = 0; r < reps + 1 && e == hipSuccess; r++) {
        float ms = 0.0f;
        (void)hipEventRecord(ev.a, nullptr);
        hipLaunchKernelGGL(qr::probe_read_kernel, dim3(blocks), dim3(256), 0, nullptr,
                           static_cast<const qr::u4_t*>(src), n16, static_cast<uint32_t*>(sink));
        (void)hipEventRecord(ev.b, nullptr);
        e = hipEventSynchronize(ev.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
        if (r > 0 && ms < best_r) best_r = ms;
        (void)hipEventRecord(ev.a, nullptr);
        hipLaunchKernelGGL(qr::probe_copy_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, nullptr,
                           static_cast<const qr::f4_t*>(src), static_cast<qr::f4_t*>(dst), n16);
        (void)hipEventRecord(ev.b, nullptr);
        if (e == hipSuccess) e = hipEventSynchronize(ev.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
        if (r > 0 && ms < best_c) best_c = ms;
    }
    if (src) (void)hipFree(src);
    if (dst) (void)hipFree(dst);
    if (sink) (void)hipFree(sink);
    if (e != hipSuccess) return -6;
    *read_gbs = (double)bytes / (best_r * 1e-3) / 1e9;
    *copy_gbs = 2.0 * (double)bytes / (best_c * 1e-3) / 1e9;
    return 0;
}

static int probe_mfma(bool rnd, uint32_t iters, int reps, double* tflops, double* clock_ghz) {
    if (!tflops || !clock_ghz) return -2;
    if (iters < 64 || iters % 4 || reps < 1) return -4;
    hipDeviceProp_t prop;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return -6;
    // four waves per CU (one per SIMD) of 4 independent chains each, 8x over
    const int blocks = prop.multiProcessorCount * 8;
    void *out = nullptr, *clk = nullptr, *tab = nullptr;
    e = hipMalloc(&out, (size_t)blocks * 256 * 4);
    if (e == hipSuccess) e = hipMalloc(&clk, (size_t)blocks * 16);
    if (e == hipSuccess && rnd) {  // 8 fragments per thread of a 256-thread block, fixed LCG
        const size_t n = 256 * 8 * 8;
        _Float16* h = new _Float16[n];
        uint32_t x = 12345u;
        for (size_t i = 0; i < n; i++) {
            x = x * 1664525u + 1013904223u;
            h[i] = (_Float16)((float)(x >> 8) * (2.0f / 16777216.0f) - 1.0f);
        }
        e = hipMalloc(&tab, n * 2);
        if (e == hipSuccess) e = hipMemcpy(tab, h, n * 2, hipMemcpyHostToDevice);
        delete[] h;
    }
    Events ev;
    float best = 1e30f;
    for (int r = 0; r < reps + 1 && e == hipSuccess; r++) {
        float ms = 0.0f;
        (void)hipEventRecord(ev.a, nullptr);
        if (rnd)
            hipLaunchKernelGGL(qr::probe_mfma_kernel<true>, dim3(blocks), dim3(256), 0, nullptr,
                               static_cast<float*>(out), iters, static_cast<unsigned long long*>(clk),
                               static_cast<const qr::h8_t*>(tab));
        else
            hipLaunchKernelGGL(qr::probe_mfma_kernel<false>, dim3(blocks), dim3(256), 0, nullptr,
                               static_cast<float*>(out), iters, static_cast<unsigned long long*>(clk),
                               static_cast<const qr::h8_t*>(tab));
        (void)hipEventRecord(ev.b, nullptr);
        e = hipEventSynchronize(ev.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
        if (r > 0 && ms < best) best = ms;
    }
    double ghz = 0.0;
    if (e == hipSuccess) {
        unsigned long long* h = new unsigned long long[(size_t)blocks * 2];
        e = hipMemcpy(h, clk, (size_t)blocks * 16, hipMemcpyDeviceToHost);
        double cyc = 0.0, real = 0.0;
        for (int b = 0; b < blocks && e == hipSuccess; b++) {
            cyc += (double)h[2 * b];
            real += (double)h[2 * b + 1];
        }
        ghz = real > 0.0 ? cyc / (real / 100e6) / 1e9 : 0.0;  // the real-time counter runs at 100 MHz
        delete[] h;
    }
    if (out) (void)hipFree(out);
    if (clk) (void)hipFree(clk);
    if (tab) (void)hipFree(tab);
    if (e != hipSuccess) return -6;
    const double flop = (double)blocks * 4 /* waves */ * qr::kChains * iters * (32.0 * 32.0 * 16.0 * 2.0);
    *tflops = flop / (best * 1e-3) / 1e12;
    *clock_ghz = ghz;
    return 0;
}

int m4_probe_mfma_f16(uint32_t iters, int reps, double* tflops, double* clock_ghz) {
    return probe_mfma(false, iters, reps, tflops, clock_ghz);
}

int m4_probe_mfma_f16_random(uint32_t iters, int reps, double* tflops, double* clock_ghz) {
    return probe_mfma(true, iters, reps, tflops, clock_ghz);
}

}  // extern "C"
