// qr_formats.h -- wire formats of the quantization router (host + device).
//
// Format ids, block layouts and the metadata table follow the reference's
// quant_router.h:14-136 (ids 0..7) and core/memory/quant_types.h:17-147
// (QUANT_CUSTOM = 99).  Layouts are byte-identical so packed weights produced
// for the reference drop in unchanged.  Weight matrices are [N, K] with the
// blocks of output column n contiguous: block (n, kb) sits at byte
// (n * (K / block_elems) + kb) * block_bytes.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace qr {

enum QuantFormat : int {
    QUANT_Q4_0 = 0,
    QUANT_MLX_4BIT = 1,
    QUANT_Q4_K = 2,
    QUANT_TERNARY_1_58 = 3,
    QUANT_VAR_RATE_AFFINE = 4,
    QUANT_EXL3 = 5,
    QUANT_Q8_0 = 6,
    QUANT_PRISM_Q2_0 = 7,
    // MLX's own 4-bit quantization, groups of 64 (mlx.core.quantize with
    // group_size 64, bits 4): one 36-byte block per group = the group's fp16
    // scale and bias followed by its eight uint32 code words exactly as MLX
    // packs them (element 8j + i in bits 4i of word j).  Not in the
    // reference, whose MLX_4BIT block is 32 elements (quant_router.h:41-45);
    // BASELINE's MLX configuration is this layout (4.5 bits per weight).
    QUANT_MLX_4BIT_G64 = 8,
    QUANT_CUSTOM = 99,
};

enum LayoutMode : int { LAYOUT_STANDARD = 0, LAYOUT_DIRECT_HEAD = 1 };

// Scales are stored as raw binary16 bits so one header serves host and device.
struct block_q4_0 { uint16_t d; uint8_t qs[16]; };
struct block_mlx_4bit { uint16_t d; uint16_t bias; uint8_t qs[16]; };
struct block_q4_K { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct block_ternary_1_58 { uint16_t d; uint16_t _pad; uint32_t qs[2]; };
struct block_var_rate_affine {
    uint16_t d; uint16_t bias; uint8_t scales[8]; uint8_t biases[8]; uint8_t modes[8];
    uint8_t _pad[4]; uint8_t qs[128];
};
struct block_exl3 {
    uint16_t d; uint16_t bias; uint8_t scales[8]; uint8_t residuals[8]; int8_t codebook[16];
    uint8_t _pad[12]; uint8_t qs[96];
};
struct block_q8_0 { uint16_t d; int8_t qs[32]; };
struct block_prism_q2_0 { uint16_t d; uint8_t qs[32]; };
struct block_mlx_4bit_g64 { uint16_t scale; uint16_t bias; uint32_t qs[8]; };

static_assert(sizeof(block_q4_0) == 18, "Q4_0 block is 18 bytes");
static_assert(sizeof(block_mlx_4bit) == 20, "MLX_4BIT block is 20 bytes");
static_assert(sizeof(block_q4_K) == 144, "Q4_K super-block is 144 bytes");
static_assert(sizeof(block_ternary_1_58) == 12, "TERNARY block is 12 bytes");
static_assert(sizeof(block_var_rate_affine) == 160, "VAR_RATE super-block is 160 bytes");
static_assert(sizeof(block_exl3) == 144, "EXL3 super-block is 144 bytes");
static_assert(sizeof(block_q8_0) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(block_prism_q2_0) == 34, "PRISM_Q2_0 block is 34 bytes");
static_assert(sizeof(block_mlx_4bit_g64) == 36, "MLX_4BIT_G64 block is 36 bytes");

struct QuantFormatInfo {
    QuantFormat format;
    const char* name;
    const char* description;
    uint32_t block_size;   // elements per block / super-block
    uint32_t block_bytes;  // bytes per block struct
    double bits_per_weight;
};

// quant_router.h:110-130
inline QuantFormatInfo get_quant_info(QuantFormat fmt) {
    switch (fmt) {
        case QUANT_Q4_0: return {fmt, "Q4_0", "Standard 32-elem symmetric block (FP16 scale)", 32, 18, 4.50};
        case QUANT_MLX_4BIT: return {fmt, "MLX_4BIT", "MLX 32-elem affine block (FP16 scale + FP16 bias)", 32, 20, 5.00};
        case QUANT_Q4_K: return {fmt, "Q4_K", "GGUF 256-elem super-block (6-bit scales & mins)", 256, 144, 4.50};
        case QUANT_TERNARY_1_58: return {fmt, "TERNARY_1_58", "BitNet 1.58-bit 32-elem ternary {-1, 0, +1} (FP16 scale)", 32, 12, 3.00};
        case QUANT_VAR_RATE_AFFINE: return {fmt, "VAR_RATE_AFFINE", "Grouped Variable-Rate Affine 256-elem mixed 3/4/5-bit super-block", 256, 160, 5.00};
        case QUANT_EXL3: return {fmt, "EXL3", "ExLlamaV3 256-elem hierarchical vector codebook super-block with residual correction", 256, 144, 4.50};
        case QUANT_Q8_0: return {fmt, "Q8_0", "Standard 32-elem 8-bit symmetric block (FP16 scale)", 32, 34, 8.50};
        case QUANT_PRISM_Q2_0: return {fmt, "PRISM_Q2_0", "PrismML Q2_0 128-elem ternary {-1, 0, +1} block (FP16 scale)", 128, 34, 2.125};
        case QUANT_MLX_4BIT_G64: return {fmt, "MLX_4BIT_G64", "MLX 64-elem affine group (FP16 scale + FP16 bias, 8 codes per uint32)", 64, 36, 4.50};
        default: break;
    }
    return {QUANT_Q4_0, "UNKNOWN", "Unknown format", 32, 0, 0.0};
}

// quant_router.h:132-136
inline size_t compute_quant_weight_bytes(QuantFormat fmt, size_t total_elements) {
    QuantFormatInfo info = get_quant_info(fmt);
    size_t num_blocks = (total_elements + info.block_size - 1) / info.block_size;
    return num_blocks * info.block_bytes;
}

// Minimum W bytes the projection entry points accept for formats 0..5
// (core/bridge/m4_mlx_bridge.mm:58-75): whole blocks per column, no rounding up.
inline size_t expected_weight_bytes(int format, uint32_t K, uint32_t N) {
    switch (format) {
        case QUANT_Q4_0: return ((size_t)K / 32) * N * 18;
        case QUANT_MLX_4BIT: return ((size_t)K / 32) * N * 20;
        case QUANT_Q4_K: return ((size_t)K / 256) * N * 144;
        case QUANT_TERNARY_1_58: return ((size_t)K / 32) * N * 12;
        case QUANT_VAR_RATE_AFFINE: return ((size_t)K / 256) * N * 160;
        case QUANT_EXL3: return ((size_t)K / 256) * N * 144;
        default: return 0;
    }
}

// W bytes the kernels read for every format that has kernels here: formats
// 0..5 as above, plus Q8_0 weights (34 B / 32) and PRISM_Q2_0 (34 B / 128),
// which the reference reaches only through its kernel names
// (quant_router_kernels.metal:726, :904; quant_registry.mm:153), and MLX's
// native g64 groups (36 B / 64).
inline size_t kernel_weight_bytes(int format, uint32_t K, uint32_t N) {
    switch (format) {
        case QUANT_Q8_0: return ((size_t)K / 32) * N * 34;
        case QUANT_PRISM_Q2_0: return ((size_t)K / 128) * N * 34;
        case QUANT_MLX_4BIT_G64: return ((size_t)K / 64) * N * 36;
        default: return expected_weight_bytes(format, K, N);
    }
}

}  // namespace qr
