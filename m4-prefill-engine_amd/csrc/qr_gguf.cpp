// qr_gguf.cpp -- GGUF ingestion (include/m4_gguf.h): parse GGUF v2/v3 files
// (mmap) or buffers in place, expose metadata and tensors, and turn tensors
// into the router's block layouts.  Host code only.
//
// Parsing follows the GGUF container the reference's GGUFLoader reads
// (core/weights/gguf_loader.mm:205-300): magic "GGUF", version 2..3, tensor
// and metadata counts, the key/value table (types 0..12, arrays recursive),
// `general.alignment` overriding the default 32, the tensor table (name,
// dims, type, offset) and the data section at the next aligned offset.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/m4_gguf.h"

namespace {

struct Value {
    int type = M4_GGUF_UINT32;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

// Little-endian readers over a bounded cursor; any read past the end fails.
struct Cursor {
    const uint8_t* p;
    size_t size, off;
    bool take(size_t n) {
        if (n > size || off > size - n) return false;
        off += n;
        return true;
    }
    bool u8(uint8_t& v) {
        if (!take(1)) return false;
        v = p[off - 1];
        return true;
    }
    bool u16(uint16_t& v) {
        if (!take(2)) return false;
        v = (uint16_t)(p[off - 2] | (p[off - 1] << 8));
        return true;
    }
    bool u32(uint32_t& v) {
        if (!take(4)) return false;
        const uint8_t* q = p + off - 4;
        v = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
        return true;
    }
    bool u64(uint64_t& v) {
        uint32_t lo, hi;
        if (!u32(lo) || !u32(hi)) return false;
        v = (uint64_t)lo | ((uint64_t)hi << 32);
        return true;
    }
    bool str(std::string& s) {
        uint64_t n;
        if (!u64(n)) return false;
        if (n > size - off) return false;
        s.assign(reinterpret_cast<const char*>(p + off), (size_t)n);
        off += (size_t)n;
        return true;
    }
    bool value(int type, Value& v, int depth) {
        v.type = type;
        switch (type) {
            case M4_GGUF_UINT8: { uint8_t x; if (!u8(x)) return false; v.u = x; return true; }
            case M4_GGUF_INT8: { uint8_t x; if (!u8(x)) return false; v.i = (int8_t)x; return true; }
            case M4_GGUF_UINT16: { uint16_t x; if (!u16(x)) return false; v.u = x; return true; }
            case M4_GGUF_INT16: { uint16_t x; if (!u16(x)) return false; v.i = (int16_t)x; return true; }
            case M4_GGUF_UINT32: { uint32_t x; if (!u32(x)) return false; v.u = x; return true; }
            case M4_GGUF_INT32: { uint32_t x; if (!u32(x)) return false; v.i = (int32_t)x; return true; }
            case M4_GGUF_FLOAT32: {
                uint32_t x;
                if (!u32(x)) return false;
                float f;
                std::memcpy(&f, &x, 4);
                v.f = f;
                return true;
            }
            case M4_GGUF_BOOL: { uint8_t x; if (!u8(x)) return false; v.u = x ? 1 : 0; return true; }
            case M4_GGUF_STRING: return str(v.s);
            case M4_GGUF_ARRAY: {
                uint32_t et;
                uint64_t n;
                if (depth > 8 || !u32(et) || !u64(n)) return false;
                if (n > size - off) return false;  // every element takes >= 1 byte
                v.arr.resize((size_t)n);
                for (auto& e : v.arr)
                    if (!value((int)et, e, depth + 1)) return false;
                return true;
            }
            case M4_GGUF_UINT64: return u64(v.u);
            case M4_GGUF_INT64: { uint64_t x; if (!u64(x)) return false; v.i = (int64_t)x; return true; }
            case M4_GGUF_FLOAT64: {
                uint64_t x;
                if (!u64(x)) return false;
                std::memcpy(&v.f, &x, 8);
                return true;
            }
            default: return false;  // unknown value type
        }
    }
};

}  // namespace

struct m4_gguf {
    const uint8_t* data = nullptr;
    size_t size = 0;
    bool mapped = false;
    int fd = -1;
    uint32_t version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    std::map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> index;

    bool parse() {
        Cursor c{data, size, 0};
        if (size < 24 || std::memcmp(data, "GGUF", 4) != 0) return false;
        c.off = 4;
        if (!c.u32(version) || version < 2 || version > 3) return false;
        if (!c.u64(n_tensors) || !c.u64(n_kv)) return false;
        for (uint64_t k = 0; k < n_kv; k++) {
            std::string key;
            uint32_t t;
            Value v;
            if (!c.str(key) || !c.u32(t) || !c.value((int)t, v, 0)) return false;
            if (key == "general.alignment") alignment = v.u ? (uint32_t)v.u : 32u;
            meta[key] = std::move(v);
        }
        for (uint64_t k = 0; k < n_tensors; k++) {
            Tensor t;
            uint32_t nd;
            if (!c.str(t.name) || !c.u32(nd)) return false;
            if ((uint64_t)nd * 8 > size - c.off) return false;
            t.dims.resize(nd);
            for (auto& d : t.dims)
                if (!c.u64(d)) return false;
            if (!c.u32(t.type) || !c.u64(t.offset)) return false;
            index[t.name] = tensors.size();
            tensors.push_back(std::move(t));
        }
        data_offset = (c.off + alignment - 1) / alignment * alignment;
        if (data_offset > size && n_tensors > 0) return false;
        return true;
    }
    const Value* get(const char* key) const {
        if (!key) return nullptr;
        auto it = meta.find(key);
        return it == meta.end() ? nullptr : &it->second;
    }
    const Tensor* tensor(const char* name) const {
        if (!name) return nullptr;
        auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
    // Start of the tensor's bytes if [start, start + bytes) lies in the file.
    const uint8_t* bytes_of(const Tensor& t, uint64_t bytes) const {
        const uint64_t a = data_offset + t.offset;
        if (a < data_offset || a > size || bytes > size - a) return nullptr;
        return data + a;
    }
    ~m4_gguf() {
        if (mapped && data) munmap(const_cast<uint8_t*>(data), size);
        if (fd >= 0) ::close(fd);
    }
};

namespace {

uint64_t elements(const Tensor& t) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) n *= d;
    return t.dims.empty() ? 0 : n;
}

// Router Q4_K scale packing (cpu_gold_reference.h:121-127): sc_j in the low 6
// bits of scales[j]; min_j's low 4 bits in scales[8 + j % 4] (low nibble for
// j < 4, high for j >= 4) and its top 2 bits in scales[j] bits 6..7.
void pack_router_scales(const uint8_t sc[8], const uint8_t mn[8], uint8_t out[12]) {
    std::memset(out, 0, 12);
    for (int j = 0; j < 8; j++) {
        out[j] = (uint8_t)((sc[j] & 63) | ((mn[j] >> 4) << 6));
        out[8 + (j & 3)] |= (uint8_t)((mn[j] & 15) << (j < 4 ? 0 : 4));
    }
}

// GGML's 6-bit scale/min packing of block_q4_K (ggml get_scale_min_k4):
// j < 4: sc = s[j] & 63, m = s[j + 4] & 63; j >= 4: sc = (s[j + 4] & 15) |
// (s[j - 4] >> 6) << 4, m = (s[j + 4] >> 4) | (s[j] >> 6) << 4.
void unpack_ggml_scales(const uint8_t s[12], uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = s[j] & 63;
            mn[j] = s[j + 4] & 63;
        } else {
            sc[j] = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
            mn[j] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
    }
}

void repack_q4_k_block(const uint8_t* g, uint8_t* r) {
    uint8_t sc[8], mn[8], code[256];
    unpack_ggml_scales(g + 4, sc, mn);
    // GGML: 32-byte chunk c holds elements 64 c + l (low nibble) and 64 c + 32 + l (high)
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            const uint8_t b = g[16 + 32 * c + l];
            code[64 * c + l] = b & 15;
            code[64 * c + 32 + l] = b >> 4;
        }
    std::memcpy(r, g, 4);  // d, dmin
    pack_router_scales(sc, mn, r + 4);
    // router: sub-block s uses bytes 16 s .. 16 s + 15; byte i low nibble ->
    // element 32 s + i, high -> 32 s + 16 + i
    for (int s = 0; s < 8; s++)
        for (int i = 0; i < 16; i++)
            r[16 + 16 * s + i] = (uint8_t)(code[32 * s + i] | (code[32 * s + 16 + i] << 4));
}

}  // namespace

extern "C" {

m4_gguf* m4_gguf_open(const char* path) {
    if (!path) return nullptr;
    auto* g = new m4_gguf();
    g->fd = ::open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size < 24) {
        delete g;
        return nullptr;
    }
    g->size = (size_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_SHARED, g->fd, 0);
    if (m == MAP_FAILED) {
        g->size = 0;
        delete g;
        return nullptr;
    }
    g->data = static_cast<const uint8_t*>(m);
    g->mapped = true;
    if (!g->parse()) {
        delete g;
        return nullptr;
    }
    return g;
}

m4_gguf* m4_gguf_parse_buffer(const void* data, size_t size) {
    if (!data || size < 24) return nullptr;
    auto* g = new m4_gguf();
    g->data = static_cast<const uint8_t*>(data);
    g->size = size;
    if (!g->parse()) {
        delete g;
        return nullptr;
    }
    return g;
}

void m4_gguf_close(m4_gguf* g) { delete g; }

uint32_t m4_gguf_version(const m4_gguf* g) { return g ? g->version : 0; }
uint64_t m4_gguf_tensor_count(const m4_gguf* g) { return g ? g->n_tensors : 0; }
uint64_t m4_gguf_metadata_count(const m4_gguf* g) { return g ? g->n_kv : 0; }
uint32_t m4_gguf_alignment(const m4_gguf* g) { return g ? g->alignment : 0; }
uint64_t m4_gguf_tensor_data_offset(const m4_gguf* g) { return g ? g->data_offset : 0; }
size_t m4_gguf_file_size(const m4_gguf* g) { return g ? g->size : 0; }

bool m4_gguf_has_metadata(const m4_gguf* g, const char* key) { return g && g->get(key); }

int m4_gguf_metadata_type(const m4_gguf* g, const char* key) {
    const Value* v = g ? g->get(key) : nullptr;
    return v ? v->type : -1;
}

int64_t m4_gguf_get_string_metadata(const m4_gguf* g, const char* key, char* out, size_t cap) {
    const Value* v = g ? g->get(key) : nullptr;
    if (!v || v->type != M4_GGUF_STRING) return -1;
    if (out && cap) {
        const size_t n = v->s.size() < cap - 1 ? v->s.size() : cap - 1;
        std::memcpy(out, v->s.data(), n);
        out[n] = '\0';
    }
    return (int64_t)v->s.size();
}

// gguf_loader.mm:317-325: unsigned 32/64-bit entries only
uint32_t m4_gguf_get_uint32_metadata(const m4_gguf* g, const char* key, uint32_t def) {
    const Value* v = g ? g->get(key) : nullptr;
    return (v && (v->type == M4_GGUF_UINT32 || v->type == M4_GGUF_UINT64)) ? (uint32_t)v->u : def;
}

uint64_t m4_gguf_get_uint64_metadata(const m4_gguf* g, const char* key, uint64_t def) {
    const Value* v = g ? g->get(key) : nullptr;
    return (v && (v->type == M4_GGUF_UINT32 || v->type == M4_GGUF_UINT64)) ? v->u : def;
}

double m4_gguf_get_number_metadata(const m4_gguf* g, const char* key, double def) {
    const Value* v = g ? g->get(key) : nullptr;
    if (!v) return def;
    switch (v->type) {
        case M4_GGUF_UINT8: case M4_GGUF_UINT16: case M4_GGUF_UINT32: case M4_GGUF_UINT64: case M4_GGUF_BOOL:
            return (double)v->u;
        case M4_GGUF_INT8: case M4_GGUF_INT16: case M4_GGUF_INT32: case M4_GGUF_INT64:
            return (double)v->i;
        case M4_GGUF_FLOAT32: case M4_GGUF_FLOAT64:
            return v->f;
        default:
            return def;
    }
}

int64_t m4_gguf_get_array_length(const m4_gguf* g, const char* key) {
    const Value* v = g ? g->get(key) : nullptr;
    return (v && v->type == M4_GGUF_ARRAY) ? (int64_t)v->arr.size() : -1;
}

bool m4_gguf_has_tensor(const m4_gguf* g, const char* name) { return g && g->tensor(name); }

int m4_gguf_get_tensor_info(const m4_gguf* g, const char* name, m4_gguf_tensor_info* out) {
    const Tensor* t = g ? g->tensor(name) : nullptr;
    if (!t || !out) return -1;
    std::memset(out, 0, sizeof(*out));
    out->n_dims = (uint32_t)t->dims.size();
    for (size_t d = 0; d < t->dims.size() && d < 4; d++) out->dims[d] = t->dims[d];
    out->type = t->type;
    out->offset = t->offset;
    return 0;
}

const char* m4_gguf_tensor_name(const m4_gguf* g, uint64_t i) {
    return (g && i < g->tensors.size()) ? g->tensors[(size_t)i].name.c_str() : nullptr;
}

// gguf_loader.mm:340-347: null when the tensor starts at or past the end
const void* m4_gguf_get_tensor_raw_data(const m4_gguf* g, const char* name) {
    const Tensor* t = g ? g->tensor(name) : nullptr;
    if (!t) return nullptr;
    const uint64_t a = g->data_offset + t->offset;
    return (a < g->size) ? g->data + a : nullptr;
}

int64_t m4_gguf_extract_q2_0_tensor(const m4_gguf* g, const char* name, void* dst, size_t cap, uint64_t* out_k,
                                    uint64_t* out_n) {
    const Tensor* t = g ? g->tensor(name) : nullptr;
    if (!t) return -1;
    const uint64_t n = elements(*t);
    if (n == 0 || n % 128) return -1;
    const uint64_t blocks = n / 128;
    const uint8_t* src = g->bytes_of(*t, blocks * 34);
    if (!src || !dst || cap < blocks * 34) return -1;
    std::memcpy(dst, src, (size_t)(blocks * 34));  // {le16 d, qs[32]}: already the block layout
    if (out_k) *out_k = t->dims[0];
    if (out_n) *out_n = t->dims.size() >= 2 ? t->dims[1] : 1;
    return (int64_t)blocks;
}

int64_t m4_gguf_load_router_weights(const m4_gguf* g, const char* name, void* dst, size_t cap, int* format,
                                    uint32_t* K, uint32_t* N) {
    const Tensor* t = g ? g->tensor(name) : nullptr;
    if (!t || t->dims.empty()) return -1;
    const uint64_t k = t->dims[0];
    uint64_t n = 1;
    for (size_t d = 1; d < t->dims.size(); d++) n *= t->dims[d];
    int f;
    uint64_t be, bb;  // block elements, block bytes
    switch (t->type) {
        case M4_GGML_Q4_0: f = 0; be = 32; bb = 18; break;
        case M4_GGML_Q4_K: f = 2; be = 256; bb = 144; break;
        case M4_GGML_Q8_0: f = 6; be = 32; bb = 34; break;
        case M4_GGML_PRISM_Q2_0:
        case M4_GGML_PRISM_Q2_0_ALT: f = 7; be = 128; bb = 34; break;
        default: return -3;
    }
    if (k == 0 || k % be || k > 0xffffffffull || n > 0xffffffffull) return -4;
    const uint64_t bytes = k / be * n * bb;
    const uint8_t* src = g->bytes_of(*t, bytes);
    if (!src) return -1;
    if (format) *format = f;
    if (K) *K = (uint32_t)k;
    if (N) *N = (uint32_t)n;
    if (!dst) return (int64_t)bytes;
    if (cap < bytes) return -2;
    if (f == 2) {
        m4_repack_ggml_q4_k(src, (size_t)(bytes / 144), dst);
    } else {
        std::memcpy(dst, src, (size_t)bytes);
    }
    return (int64_t)bytes;
}

int m4_repack_ggml_q4_k(const void* src, size_t num_blocks, void* dst) {
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* d = static_cast<uint8_t*>(dst);
    for (size_t b = 0; b < num_blocks; b++) repack_q4_k_block(s + 144 * b, d + 144 * b);
    return 0;
}

int m4_repack_mlx_g64(const void* wq, const void* scales, const void* biases, uint32_t N, uint32_t K, void* dst) {
    if (K % 64) return -4;
    const uint32_t* q = static_cast<const uint32_t*>(wq);
    const uint16_t* sc = static_cast<const uint16_t*>(scales);
    const uint16_t* bi = static_cast<const uint16_t*>(biases);
    uint8_t* out = static_cast<uint8_t*>(dst);
    const uint32_t groups = K / 64, words = K / 8;
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t b = 0; b < K / 32; b++) {
            uint8_t* blk = out + ((size_t)n * (K / 32) + b) * 20;
            const uint16_t s = sc[(size_t)n * groups + b / 2], c = bi[(size_t)n * groups + b / 2];
            std::memcpy(blk, &s, 2);
            std::memcpy(blk + 2, &c, 2);
            const uint32_t* w = q + (size_t)n * words + 4 * b;  // elements 32 b .. 32 b + 31
            auto code = [&](int e) { return (uint8_t)((w[e >> 3] >> (4 * (e & 7))) & 15u); };
            for (int i = 0; i < 16; i++) blk[4 + i] = (uint8_t)(code(i) | (code(i + 16) << 4));
        }
    return 0;
}

}  // extern "C"
