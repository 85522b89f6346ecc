// qr_device.h -- gfx950 device helpers shared by the router kernels.
//
// Vector types for CDNA4 MFMA operands, buffer-resource loads (bounds-checked
// in hardware: an offset past num_records reads 0, which the kernels use for
// ragged M/N edges), and exact fp16 rounding helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qr {


typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16v_t __attribute__((ext_vector_type(16)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

// Third dword of a raw buffer descriptor on gfx9-family parts (32-bit data
// format, untyped access); num_records is a byte count.
constexpr int kBufferFlags = 0x00020000;
// An offset that is always past num_records: loads from it return 0.
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}
__device__ __forceinline__ uint32_t ld_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ u2_t ld_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ u4_t ld_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Bit casts through by-value parameters.  (This toolchain's clang miscompiles
// __builtin_bit_cast applied directly to an ext_vector element such as v.y:
// every element reads as element 0.)
__device__ __forceinline__ uint32_t f32_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t as_u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t f2h_bits(float x) {  // RNE (v_cvt_f16_f32)
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ uint32_t pack_h2(uint32_t lo16, uint32_t hi16) { return lo16 | (hi16 << 16); }

// Round-to-nearest-even binary16 of the EXACT sum p + q of two floats.
// The float sum s is made round-to-odd with its TwoSum error term; RNE of a
// round-to-odd value with >= 2 extra bits equals RNE of the exact value.
__device__ __forceinline__ uint32_t rne16_sum(float p, float q) {
    float s = p + q;
    float bb = s - p;
    float err = (p - (s - bb)) + (q - bb);
    uint32_t bits = __builtin_bit_cast(uint32_t, s);
    if (err != 0.0f && !(bits & 1u)) {
        bool away = (err > 0.0f) == (s > 0.0f);
        bits = away ? bits + 1u : bits - 1u;
    }
    return f2h_bits(__builtin_bit_cast(float, bits));
}

// Byte permute: D.byte[i] = sel.byte[i] in 0..3 -> s1.byte, 4..7 -> s0.byte, 0x0c -> 0.
// SiLU(g) * u in fp32 for the SwiGLU epilogues: g / (1 + e^-g) through the
// hardware reciprocal (about 1 ulp of fp32, far inside the fp16 result's
// rounding) instead of an IEEE division sequence; e^-g = inf gives -0 and
// e^-g = 0 gives g, as the division does.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

// Two 4-bit codes from bytes 0/1 (or 2/3) of a nibble-per-byte word, as the
// binary16 pair {1024 + c0, 1024 + c1} (magic-exponent conversion: exact).
__device__ __forceinline__ uint32_t nib_pair_lo(uint32_t x) { return perm(0x64646464u, x, 0x04010400u); }
__device__ __forceinline__ uint32_t nib_pair_hi(uint32_t x) { return perm(0x64646464u, x, 0x04030402u); }

// {q0, q1} from a magic pair {1024 + q0, 1024 + q1}: exact halves.
__device__ __forceinline__ h2_t magic_to_q(uint32_t magic_pair) {
    const h2_t off = {(_Float16)1024.0f, (_Float16)1024.0f};
    return as_h2(magic_pair) - off;
}

// Exact binary16 pair {c0, c1} of two codes 0..15 held one per byte, in bytes
// 0, 1 (HI = false) or 2, 3 (HI = true) of a word.  A byte c read as an OCP
// e4m3 value is c * 2^-9 for every c in 0..15 (subnormal for c < 8, exponent
// field 1 for c >= 8: the two ranges join linearly), so the scaled conversion
// by 2^9 is exact -- one packed instruction per pair.
template <bool HI>
__device__ __forceinline__ h2_t code_pair(uint32_t bytes) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(bytes, 512.0f, HI);
}

// Largest |d| for which -8 d is finite in binary16 (65504 / 8).
constexpr float kQ4_0FastMaxScale = 8188.0f;

// RNE binary16 of q*A + C for both codes of a pair, when q*A + C is exact in
// fp32 (fused fp32 fma of the fp16 code, one rounding to fp16).  Built as a
// half2 vector so the pair is one v_fma_mixlo_f16 + one v_fma_mixhi_f16 into
// the same register (two separate halves cost a shift and an OR more).
__device__ __forceinline__ uint32_t affine_pair_exact(h2_t q, float A, float C) {
    const h2_t r = {(_Float16)__builtin_fmaf((float)q.x, A, C), (_Float16)__builtin_fmaf((float)q.y, A, C)};
    return __builtin_bit_cast(uint32_t, r);
}

// Same for any inputs: the exact-sum (round-to-odd) path where `exact` is false.
__device__ __forceinline__ uint32_t affine_pair_any(h2_t q, float A, float C, bool exact) {
    const float q0 = (float)q.x, q1 = (float)q.y;
    const uint32_t lo = exact ? f2h_bits(__builtin_fmaf(q0, A, C)) : rne16_sum(q0 * A, C);
    const uint32_t hi = exact ? f2h_bits(__builtin_fmaf(q1, A, C)) : rne16_sum(q1 * A, C);
    return lo | (hi << 16);
}


// Raises a kernel's dynamic-LDS limit to `bytes` once per device (HIP function
// attributes are per device); `done` is the caller's per-kernel record.
constexpr int kMaxDevices = 64;
inline hipError_t lds_limit_once(const void* kern, size_t bytes, size_t (&done)[kMaxDevices]) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    if (done[dev] >= bytes) return hipSuccess;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) done[dev] = bytes;
    return e;
}

}  // namespace qr
