// qr_registry.h -- host codec registry (src/router/quant_registry.h:14-65).
//
// A process-wide map from format id to codec descriptor with the reference's
// names, block sizes, struct sizes, bits/weight and kernel symbol names, plus
// runtime registration (QUANT_CUSTOM = 99 and friends).
#pragma once
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "qr_formats.h"

namespace qr {

struct QuantCodecDescriptor {
    QuantFormat format;
    std::string name;
    std::string description;
    uint32_t block_size;
    size_t struct_size;
    double bits_per_weight;
    std::string gemm_kernel_name;
    std::string head_gemm_kernel_name;
    std::function<void(const void* src, void* dst, size_t count)> quantize_fn;
    std::function<void(const void* src, float* dst, size_t count)> dequantize_fn;
};

class QuantRegistry {
public:
    static QuantRegistry& instance();
    void register_codec(const QuantCodecDescriptor& desc);
    const QuantCodecDescriptor* get(QuantFormat format) const;
    const QuantCodecDescriptor* get_by_name(const std::string& name) const;
    std::vector<QuantFormat> available_formats() const;
    size_t compute_weight_bytes(QuantFormat format, size_t num_elements) const;
    bool has_format(QuantFormat format) const;

private:
    QuantRegistry();
    void register_builtin_codecs();
    mutable std::mutex mu_;
    std::map<QuantFormat, QuantCodecDescriptor> registry_;
    std::map<std::string, QuantFormat> name_to_format_;
};

struct CodecRegistrationHelper {
    explicit CodecRegistrationHelper(const QuantCodecDescriptor& desc) { QuantRegistry::instance().register_codec(desc); }
};

#define QR_CONCAT_INNER(a, b) a##b
#define QR_CONCAT(a, b) QR_CONCAT_INNER(a, b)
#define REGISTER_QUANT_CODEC(...) \
    static ::qr::CodecRegistrationHelper QR_CONCAT(_qr_codec_reg_, __LINE__)(__VA_ARGS__);

}  // namespace qr
