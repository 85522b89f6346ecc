// qr_registry.cpp -- built-in codecs of the router (src/router/quant_registry.mm:60-172).
#include "qr_registry.h"

#include <cstring>

#include "../../include/m4_mlx_bridge.h"

namespace qr {

QuantRegistry& QuantRegistry::instance() {
    static QuantRegistry reg;
    return reg;
}

QuantRegistry::QuantRegistry() { register_builtin_codecs(); }

void QuantRegistry::register_codec(const QuantCodecDescriptor& desc) {
    std::lock_guard<std::mutex> lk(mu_);
    registry_[desc.format] = desc;
    name_to_format_[desc.name] = desc.format;
}

const QuantCodecDescriptor* QuantRegistry::get(QuantFormat format) const {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = registry_.find(format);
    return it == registry_.end() ? nullptr : &it->second;
}

const QuantCodecDescriptor* QuantRegistry::get_by_name(const std::string& name) const {
    QuantFormat f;
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = name_to_format_.find(name);
        if (it == name_to_format_.end()) return nullptr;
        f = it->second;
    }
    return get(f);
}

std::vector<QuantFormat> QuantRegistry::available_formats() const {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<QuantFormat> v;
    v.reserve(registry_.size());
    for (const auto& kv : registry_) v.push_back(kv.first);
    return v;
}

bool QuantRegistry::has_format(QuantFormat format) const {
    std::lock_guard<std::mutex> lk(mu_);
    return registry_.count(format) != 0;
}

size_t QuantRegistry::compute_weight_bytes(QuantFormat format, size_t num_elements) const {
    const auto* d = get(format);
    if (!d || d->block_size == 0) return 0;
    return (num_elements + d->block_size - 1) / d->block_size * d->struct_size;
}

void QuantRegistry::register_builtin_codecs() {
    struct Row { QuantFormat f; const char* desc; const char* sym; };
    // Descriptions and kernel symbol names as registered by the reference
    // (quant_registry.mm:62-171); sizes from the wire-format table.
    const Row rows[] = {
        {QUANT_Q4_0, "Standard GGUF Q4_0 Symmetric 32-element blocks", "q4_0"},
        {QUANT_MLX_4BIT, "MLX-style 4-bit affine with grouped scale and bias", "mlx_4bit"},
        {QUANT_Q4_K, "GGUF Q4_K super-block with 8x32 sub-blocks", "q4_k"},
        {QUANT_TERNARY_1_58, "BitNet 1.58-bit ternary {-1, 0, +1} packed weights", "ternary_1_58"},
        {QUANT_VAR_RATE_AFFINE, "Grouped Variable-Rate Affine 256-elem mixed 3/4/5-bit super-block", "var_rate_affine"},
        {QUANT_EXL3, "ExLlamaV3 256-elem super-block with vector codebook", "exl3"},
        {QUANT_Q8_0, "Standard GGUF Q8_0 Symmetric 32-element blocks (for KV cache)", "q8_0"},
        {QUANT_PRISM_Q2_0, "PrismML Q2_0 128-elem ternary {-1, 0, +1} block (FP16 scale)", "prism_q2_0"},
        // not registered by the reference: MLX's native 64-element groups
        {QUANT_MLX_4BIT_G64, "MLX 4-bit affine, native 64-element groups (8 codes per uint32)", "mlx_4bit_g64"},
    };
    for (const auto& r : rows) {
        QuantFormatInfo info = get_quant_info(r.f);
        QuantCodecDescriptor d;
        d.format = r.f;
        d.name = info.name;
        d.description = r.desc;
        d.block_size = info.block_size;
        d.struct_size = info.block_bytes;
        d.bits_per_weight = info.bits_per_weight;
        d.gemm_kernel_name = std::string("quant_router_gemm_") + r.sym + "_64x64";
        d.head_gemm_kernel_name = std::string("quant_router_head_gemm_") + r.sym + "_64x64";
        register_codec(d);
    }
}

}  // namespace qr

// ---------------------------------------------------------------------------
// C-ABI view of the registry
// ---------------------------------------------------------------------------
extern "C" {

int m4_registry_get(int format, m4_quant_codec_info* out) {
    const auto* d = qr::QuantRegistry::instance().get(static_cast<qr::QuantFormat>(format));
    if (!d || !out) return -3;
    out->format = d->format;
    out->name = d->name.c_str();
    out->description = d->description.c_str();
    out->block_size = d->block_size;
    out->struct_size = d->struct_size;
    out->bits_per_weight = d->bits_per_weight;
    out->gemm_kernel_name = d->gemm_kernel_name.c_str();
    out->head_gemm_kernel_name = d->head_gemm_kernel_name.c_str();
    return 0;
}

int m4_registry_get_by_name(const char* name) {
    if (!name) return -3;
    const auto* d = qr::QuantRegistry::instance().get_by_name(name);
    return d ? static_cast<int>(d->format) : -3;
}

int m4_registry_available_formats(int* out, int cap) {
    auto v = qr::QuantRegistry::instance().available_formats();
    for (int i = 0; i < (int)v.size() && i < cap && out; i++) out[i] = static_cast<int>(v[i]);
    return (int)v.size();
}

uint64_t m4_registry_compute_weight_bytes(int format, uint64_t num_elements) {
    return qr::QuantRegistry::instance().compute_weight_bytes(static_cast<qr::QuantFormat>(format), num_elements);
}

bool m4_registry_has_format(int format) {
    return qr::QuantRegistry::instance().has_format(static_cast<qr::QuantFormat>(format));
}

int m4_registry_register_codec(const m4_quant_codec_info* info) {
    if (!info || !info->name) return -2;
    qr::QuantCodecDescriptor d;
    d.format = static_cast<qr::QuantFormat>(info->format);
    d.name = info->name;
    d.description = info->description ? info->description : "";
    d.block_size = info->block_size;
    d.struct_size = info->struct_size;
    d.bits_per_weight = info->bits_per_weight;
    d.gemm_kernel_name = info->gemm_kernel_name ? info->gemm_kernel_name : "";
    d.head_gemm_kernel_name = info->head_gemm_kernel_name ? info->head_gemm_kernel_name : "";
    qr::QuantRegistry::instance().register_codec(d);
    return 0;
}

}  // extern "C"
