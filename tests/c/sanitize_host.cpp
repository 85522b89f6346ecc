// Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).
//
// Built by tests/test_sanitizers.py with -fsanitize=address,undefined
// -fno-sanitize-recover=all together with the host-only sources of the
// library (qr_gguf.cpp, qr_registry.cpp, qr_host.cpp) and the CPU oracle
// (oracle/oracle.c).  It drives the code that reads untrusted bytes or
// caller-sized buffers:
//  * the GGUF parser, on well-formed files and on every truncation, seeded
//    byte flips and garbage, each parsed from a heap copy of exactly its size
//    (a read past the end is an ASan report) and, for a few, from disk;
//  * the GGUF router-weight loader and repacks, with exact-size destinations;
//  * the registry's C view;
//  * argument validation and the host-range probe (a guard page included);
//  * every oracle entry point on small inputs of every format.
// Exit status 0 and "sanitize_host: ok" = no report (a report aborts).
#include <sys/mman.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/m4_gguf.h"
#include "../../include/m4_mlx_bridge.h"
#include "../../m4-prefill-engine_amd/csrc/qr_host.h"

extern "C" {
uint32_t orc_block_elems(int f);
uint32_t orc_block_bytes(int f);
int orc_dequantize(int f, const uint8_t* W, uint16_t* out, uint32_t K, uint32_t N);
int orc_dequantize_f64(int f, const uint8_t* W, double* out, uint32_t K, uint32_t N);
int orc_gemm(int f, const uint16_t* A, const uint8_t* B, uint16_t* C, const uint16_t* R, uint32_t M, uint32_t N,
             uint32_t K, int direct_head, uint32_t H, uint32_t D, int nthreads);
int orc_swiglu(int f, const uint16_t* A, const uint8_t* Bg, const uint8_t* Bu, uint16_t* O, uint32_t M, uint32_t N,
               uint32_t K, int nthreads);
void orc_quantize_q8_0(const uint16_t* src, uint8_t* dst, size_t num_blocks);
void orc_dequantize_q8_0(const uint8_t* src, uint16_t* dst, size_t num_blocks);
void orc_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O, uint32_t H, uint32_t M,
                   uint32_t D, float scale, int o_token_major, int nthreads);
int orc_attention_gqa(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O, uint32_t H, uint32_t Hkv,
                      uint32_t M, uint32_t D, float scale, int o_token_major, int nthreads);
int orc_attention_rows(const uint16_t* Qr, const uint16_t* K, const uint16_t* V, uint16_t* Or, const uint32_t* pos,
                       uint32_t nr, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D, float scale, int o_token_major,
                       int nthreads);
void orc_attention_q8_0(const uint16_t* Q, const uint8_t* Kq, const uint8_t* Vq, uint16_t* O, uint32_t H, uint32_t M,
                        uint32_t D, float scale, int o_token_major, int nthreads);
int orc_attention_q8_0_gqa(const uint16_t* Q, const uint8_t* Kq, const uint8_t* Vq, uint16_t* O, uint32_t H,
                           uint32_t Hkv, uint32_t M, uint32_t D, float scale, int o_token_major, int nthreads);
int orc_rmsnorm(const uint16_t* X, const uint16_t* w, uint16_t* Y, uint32_t M, uint32_t D, float eps, int norm_type);
int orc_rope(uint16_t* T, uint32_t H, uint32_t M, uint32_t D, float theta, uint32_t offset, int traditional);
int orc_layer(int f, const uint16_t* X, const uint8_t* Wq, const uint8_t* Wk, const uint8_t* Wv, const uint8_t* Wo,
              const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, uint16_t* Xout, uint32_t M, uint32_t dm,
              uint32_t H, uint32_t D, uint32_t Nm, float scale, uint16_t* Qh, uint16_t* Kh, uint16_t* Vh,
              uint16_t* Oattn, uint16_t* Xmid, uint16_t* S, int nthreads);
int orc_layer_ex(int f, const uint16_t* X, const uint16_t* w_attn, const uint8_t* Wq, const uint8_t* Wk,
                 const uint8_t* Wv, const uint8_t* Wo, const uint16_t* w_ffn, const uint8_t* Wg, const uint8_t* Wu,
                 const uint8_t* Wd, uint16_t* Xout, uint32_t M, uint32_t dm, uint32_t Hq, uint32_t Hkv, uint32_t D,
                 uint32_t Nm, float scale, int norm_type, float eps, int rope, float theta, uint32_t offset,
                 int traditional, int nthreads);
int orc_layer_ex_rows(int f, const uint16_t* X, const uint16_t* w_attn, const uint8_t* Wq, const uint8_t* Wk,
                      const uint8_t* Wv, const uint8_t* Wo, const uint16_t* w_ffn, const uint8_t* Wg,
                      const uint8_t* Wu, const uint8_t* Wd, uint16_t* Xout, const uint32_t* pos, uint32_t nr,
                      uint32_t M, uint32_t dm, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t Nm, float scale,
                      int norm_type, float eps, int rope, float theta, uint32_t offset, int traditional,
                      int nthreads);
}

#define CHECK(c)                                                            \
    do {                                                                    \
        if (!(c)) {                                                         \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);    \
            exit(1);                                                        \
        }                                                                   \
    } while (0)

static uint64_t g_rng = 0x9e3779b97f4a7c15ull;
static uint32_t rnd() {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (uint32_t)(g_rng >> 11);
}
static std::vector<uint8_t> rand_bytes(size_t n) {
    std::vector<uint8_t> v(n);
    for (auto& b : v) b = (uint8_t)rnd();
    return v;
}
// fp16 values in about [-1, 1] (exponent <= 14)
static std::vector<uint16_t> rand_f16(size_t n) {
    std::vector<uint16_t> v(n);
    for (auto& h : v) h = (uint16_t)((rnd() & 0x83ff) | ((10 + rnd() % 5) << 10));
    return v;
}
// Weight blocks of format f with finite fp16 scales (the scale fields the
// oracle reads are rewritten per format below; other bytes are random).
static std::vector<uint8_t> rand_blocks(int f, uint32_t N, uint32_t K) {
    const uint32_t bs = orc_block_elems(f), bb = orc_block_bytes(f);
    std::vector<uint8_t> w = rand_bytes((size_t)N * (K / bs) * bb);
    for (size_t b = 0; b < w.size() / bb; b++) {
        uint8_t* p = &w[b * bb];
        // every 16-bit field at an even offset of the first 4 bytes: a small fp16
        for (int o = 0; o + 1 < 4 && o + 1 < (int)bb; o += 2) {
            const uint16_t h = (uint16_t)((rnd() & 0x83ff) | ((5 + rnd() % 8) << 10));
            memcpy(p + o, &h, 2);
        }
    }
    return w;
}

// ---------------------------------------------------------------- GGUF writer
struct Writer {
    std::vector<uint8_t> b;
    void u8(uint8_t v) { b.push_back(v); }
    void u32(uint32_t v) { for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i))); }
    void u64(uint64_t v) { for (int i = 0; i < 8; i++) b.push_back((uint8_t)(v >> (8 * i))); }
    void str(const std::string& s) { u64(s.size()); b.insert(b.end(), s.begin(), s.end()); }
};
struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    std::vector<uint8_t> data;
};
// GGUF value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
// 8 string, 9 array, 10 u64, 11 i64, 12 f64.
static std::vector<uint8_t> make_gguf(const std::vector<Tensor>& ts, uint32_t align) {
    Writer w;
    w.u32(0x46554747u);  // "GGUF"
    w.u32(3);
    w.u64(ts.size());
    w.u64(9);
    w.str("general.architecture"); w.u32(8); w.str("sanitize");
    w.str("general.alignment"); w.u32(4); w.u32(align);
    w.str("a.u8"); w.u32(0); w.u8(7);
    w.str("a.i16"); w.u32(3); w.u8(0xfe); w.u8(0xff);
    w.str("a.f32"); w.u32(6); w.u32(0x3fc00000u);
    w.str("a.bool"); w.u32(7); w.u8(1);
    w.str("a.u64"); w.u32(10); w.u64(1ull << 40);
    w.str("a.f64"); w.u32(12); w.u64(0x3fb999999999999aull);
    w.str("a.arr"); w.u32(9); w.u32(9); w.u64(2);  // array of two arrays of strings
    for (int i = 0; i < 2; i++) { w.u32(8); w.u64(2); w.str("x"); w.str("yz"); }
    uint64_t off = 0;
    for (const auto& t : ts) {
        w.str(t.name);
        w.u32((uint32_t)t.dims.size());
        for (auto d : t.dims) w.u64(d);
        w.u32(t.type);
        w.u64(off);
        off += (t.data.size() + align - 1) / align * align;
    }
    while (w.b.size() % align) w.u8(0);
    for (const auto& t : ts) {
        w.b.insert(w.b.end(), t.data.begin(), t.data.end());
        while (w.b.size() % align) w.u8(0);
    }
    return w.b;
}

// Every query on a parsed file; exact-size destinations.
static void exercise(m4_gguf* g) {
    if (!g) return;
    (void)m4_gguf_version(g);
    (void)m4_gguf_alignment(g);
    (void)m4_gguf_tensor_data_offset(g);
    (void)m4_gguf_file_size(g);
    (void)m4_gguf_metadata_count(g);
    const char* keys[] = {"general.architecture", "general.alignment", "a.u8", "a.i16", "a.f32", "a.bool",
                          "a.u64", "a.f64", "a.arr", "missing"};
    for (const char* k : keys) {
        (void)m4_gguf_has_metadata(g, k);
        (void)m4_gguf_metadata_type(g, k);
        char buf[8];
        (void)m4_gguf_get_string_metadata(g, k, buf, sizeof buf);
        (void)m4_gguf_get_string_metadata(g, k, nullptr, 0);
        (void)m4_gguf_get_uint32_metadata(g, k, 3);
        (void)m4_gguf_get_uint64_metadata(g, k, 3);
        (void)m4_gguf_get_number_metadata(g, k, 0.5);
        (void)m4_gguf_get_array_length(g, k);
    }
    const uint64_t nt = m4_gguf_tensor_count(g);
    for (uint64_t i = 0; i < nt + 1; i++) {
        const char* name = m4_gguf_tensor_name(g, i);
        if (!name) continue;
        m4_gguf_tensor_info info;
        (void)m4_gguf_get_tensor_info(g, name, &info);
        (void)m4_gguf_has_tensor(g, name);
        (void)m4_gguf_get_tensor_raw_data(g, name);
        int fmt = -1;
        uint32_t K = 0, N = 0;
        const int64_t need = m4_gguf_load_router_weights(g, name, nullptr, 0, &fmt, &K, &N);
        if (need > 0 && need < (int64_t)(64 << 20)) {
            std::vector<uint8_t> dst((size_t)need);
            CHECK(m4_gguf_load_router_weights(g, name, dst.data(), dst.size(), &fmt, &K, &N) == need);
            if (need > 1) CHECK(m4_gguf_load_router_weights(g, name, dst.data(), dst.size() - 1, &fmt, &K, &N) == -2);
        }
        uint64_t k2 = 0, n2 = 0;
        const int64_t nb = m4_gguf_extract_q2_0_tensor(g, name, nullptr, 0, &k2, &n2);
        if (nb > 0 && nb < (1 << 20)) {
            std::vector<uint8_t> dst((size_t)nb * 34);
            (void)m4_gguf_extract_q2_0_tensor(g, name, dst.data(), dst.size(), &k2, &n2);
        }
    }
    m4_gguf_close(g);
}

static void gguf_cases() {
    // tensors of the router types: Q4_0 (2), Q8_0 (8), Q4_K (12), PrismML Q2_0 (100), F16 (1)
    std::vector<Tensor> ts;
    ts.push_back({"t.q4_0", {64, 4}, 2, rand_bytes(4 * 2 * 18)});
    ts.push_back({"t.q8_0", {64, 3}, 8, rand_bytes(3 * 2 * 34)});
    ts.push_back({"t.q4_k", {256, 2}, 12, rand_bytes(2 * 144)});
    ts.push_back({"t.prism", {128, 2}, 100, rand_bytes(2 * 34)});
    ts.push_back({"t.f16", {8}, 1, rand_bytes(16)});
    ts.push_back({"t.odd", {33, 2}, 2, rand_bytes(40)});  // not a whole number of blocks
    for (uint32_t align : {32u, 64u}) {
        const std::vector<uint8_t> file = make_gguf(ts, align);
        // whole file, every truncation, from exact-size heap copies
        for (size_t len = 0; len <= file.size(); len++) {
            std::vector<uint8_t> cut(file.begin(), file.begin() + (long)len);
            uint8_t* heap = (uint8_t*)malloc(len ? len : 1);
            if (len) memcpy(heap, cut.data(), len);
            exercise(m4_gguf_parse_buffer(heap, len));
            free(heap);
        }
        // seeded byte flips and bit flips of the whole file
        for (int it = 0; it < 3000; it++) {
            std::vector<uint8_t> m = file;
            const int nflip = 1 + (int)(rnd() % 4);
            for (int f = 0; f < nflip; f++) {
                const size_t at = rnd() % m.size();
                m[at] = (rnd() & 1) ? (uint8_t)rnd() : (uint8_t)(m[at] ^ (1u << (rnd() % 8)));
            }
            uint8_t* heap = (uint8_t*)malloc(m.size());
            memcpy(heap, m.data(), m.size());
            exercise(m4_gguf_parse_buffer(heap, m.size()));
            free(heap);
        }
        // from disk (the mmap path)
        char path[] = "/tmp/sanitize_gguf_XXXXXX";
        const int fd = mkstemp(path);
        CHECK(fd >= 0);
        CHECK(write(fd, file.data(), file.size()) == (ssize_t)file.size());
        close(fd);
        m4_gguf* g = m4_gguf_open(path);
        CHECK(g != nullptr);
        exercise(g);
        unlink(path);
    }
    // garbage with a valid magic and version, and pure garbage
    for (int it = 0; it < 3000; it++) {
        std::vector<uint8_t> m = rand_bytes(1 + rnd() % 512);
        if (it % 2 == 0 && m.size() >= 8) {
            const uint32_t magic = 0x46554747u, ver = 2 + rnd() % 2;
            memcpy(m.data(), &magic, 4);
            memcpy(m.data() + 4, &ver, 4);
        }
        uint8_t* heap = (uint8_t*)malloc(m.size());
        memcpy(heap, m.data(), m.size());
        exercise(m4_gguf_parse_buffer(heap, m.size()));
        free(heap);
    }
    exercise(m4_gguf_parse_buffer(nullptr, 0));
    CHECK(m4_gguf_open("/nonexistent/sanitize.gguf") == nullptr);
    // repacks with exact-size buffers
    std::vector<uint8_t> src = rand_bytes(3 * 144), dst(3 * 144);
    CHECK(m4_repack_ggml_q4_k(src.data(), 3, dst.data()) == 0);
    const uint32_t N = 3, K = 128;
    std::vector<uint32_t> wq(N * K / 8);
    for (auto& x : wq) x = rnd();
    std::vector<uint16_t> sc = rand_f16(N * K / 64), bi = rand_f16(N * K / 64);
    std::vector<uint8_t> out((size_t)N * K / 32 * 20);
    CHECK(m4_repack_mlx_g64(wq.data(), sc.data(), bi.data(), N, K, out.data()) == 0);
    CHECK(m4_repack_mlx_g64(wq.data(), sc.data(), bi.data(), N, 96, out.data()) == -4);
}

// -------------------------------------------------------------- registry view
static void registry_cases() {
    int fmts[32];
    const int n = m4_registry_available_formats(fmts, 32);
    CHECK(n > 0);
    CHECK(m4_registry_available_formats(fmts, 1) >= 1);
    for (int f = -2; f < 120; f++) {
        m4_quant_codec_info info;
        if (m4_registry_get(f, &info) == 0) {
            CHECK(m4_registry_has_format(f));
            CHECK(m4_registry_get_by_name(info.name) == f);
        }
        (void)m4_registry_compute_weight_bytes(f, 4096);
        (void)m4_registry_compute_weight_bytes(f, 0);
    }
    CHECK(m4_registry_get_by_name("no_such_codec") < 0);
    CHECK(m4_registry_get_by_name("") < 0);
}

// -------------------------------------------- validation and the host probe
static void host_cases() {
    static char X[64 * 128 * 2], W[128 / 32 * 64 * 144], Y[64 * 64 * 2];
    for (int f = -1; f < 12; f++)
        for (uint32_t K : {0u, 32u, 64u, 100u, 128u, 256u})
            for (uint32_t M : {0u, 1u, 64u})
                for (bool ext : {false, true}) {
                    (void)qr::validate(X, sizeof X, W, sizeof W, Y, sizeof Y, f, M, K, 64, ext);
                    (void)qr::validate(X + 1, sizeof X, W, sizeof W, Y, sizeof Y, f, M, K, 64, ext);
                    (void)qr::validate(nullptr, 0, W, sizeof W, Y, sizeof Y, f, M, K, 64, ext);
                }
    CHECK(qr::validate(X, sizeof X, W, sizeof W, Y, sizeof Y, 0, 64, 128, 64) == 0);
    const long pg = sysconf(_SC_PAGESIZE);
    uint8_t* m = (uint8_t*)mmap(nullptr, 3 * pg, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    CHECK(m != MAP_FAILED);
    CHECK(mprotect(m + 2 * pg, pg, PROT_NONE) == 0);
    CHECK(mprotect(m + pg, pg, PROT_READ) == 0);
    CHECK(qr::host_range_ok(m, pg, true));
    CHECK(qr::host_range_ok(m, 2 * pg, false));
    CHECK(!qr::host_range_ok(m, 2 * pg, true));        // read-only page
    CHECK(!qr::host_range_ok(m, 3 * pg, false));       // guard page
    CHECK(!qr::host_range_ok(m + 2 * pg - 1, 2, false));
    CHECK(qr::host_range_ok(m, 0, true));
    std::vector<uint8_t> heap(1000);
    CHECK(qr::host_range_ok(heap.data(), heap.size(), true));
    munmap(m, 3 * pg);
}

// -------------------------------------------------------------------- oracle
static void oracle_cases() {
    const int formats[] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
    const uint32_t M = 5, N = 7, K = 256;
    for (int f : formats) {
        if (orc_block_elems(f) == 0) continue;
        std::vector<uint8_t> W = rand_blocks(f, N, K), W2 = rand_blocks(f, N, K);
        std::vector<uint16_t> A = rand_f16((size_t)M * K), R = rand_f16((size_t)M * N), C((size_t)M * N);
        std::vector<uint16_t> deq((size_t)N * K);
        std::vector<double> deq64((size_t)N * K);
        CHECK(orc_dequantize(f, W.data(), deq.data(), K, N) == 0);
        CHECK(orc_dequantize_f64(f, W.data(), deq64.data(), K, N) == 0);
        CHECK(orc_gemm(f, A.data(), W.data(), C.data(), R.data(), M, N, K, 0, 0, 0, 2) == 0);
        CHECK(orc_swiglu(f, A.data(), W.data(), W2.data(), C.data(), M, N, K, 2) == 0);
    }
    {   // direct-head layout
        std::vector<uint8_t> W = rand_blocks(0, 8, 64);
        std::vector<uint16_t> A = rand_f16(3 * 64), C(3 * 8);
        CHECK(orc_gemm(0, A.data(), W.data(), C.data(), nullptr, 3, 8, 64, 1, 2, 4, 1) == 0);
    }
    CHECK(orc_gemm(99, nullptr, nullptr, nullptr, nullptr, 1, 1, 32, 0, 0, 0, 1) == -3);
    const uint32_t H = 4, Hkv = 2, Ma = 37, D = 64;
    const size_t nq = (size_t)H * Ma * D, nk = (size_t)Hkv * Ma * D;
    std::vector<uint16_t> Q = rand_f16(nq), Kx = rand_f16(nq), V = rand_f16(nq), O(nq);
    std::vector<uint8_t> Kq(nq / 32 * 34), Vq(nq / 32 * 34);
    orc_quantize_q8_0(Kx.data(), Kq.data(), nq / 32);
    orc_quantize_q8_0(V.data(), Vq.data(), nq / 32);
    std::vector<uint16_t> back(nq);
    orc_dequantize_q8_0(Kq.data(), back.data(), nq / 32);
    orc_attention(Q.data(), Kx.data(), V.data(), O.data(), H, Ma, D, 0.125f, 0, 2);
    orc_attention(Q.data(), Kx.data(), V.data(), O.data(), H, Ma, D, 0.125f, 1, 2);
    CHECK(orc_attention_gqa(Q.data(), Kx.data(), V.data(), O.data(), H, Hkv, Ma, D, 0.125f, 0, 2) == 0);
    CHECK(orc_attention_gqa(Q.data(), Kx.data(), V.data(), O.data(), H, 3, Ma, D, 0.125f, 0, 2) == -4);
    orc_attention_q8_0(Q.data(), Kq.data(), Vq.data(), O.data(), H, Ma, D, 0.125f, 0, 2);
    std::vector<uint8_t> Kq2(nk / 32 * 34), Vq2(nk / 32 * 34);
    orc_quantize_q8_0(Kx.data(), Kq2.data(), nk / 32);
    orc_quantize_q8_0(V.data(), Vq2.data(), nk / 32);
    CHECK(orc_attention_q8_0_gqa(Q.data(), Kq2.data(), Vq2.data(), O.data(), H, Hkv, Ma, D, 0.125f, 1, 2) == 0);
    const uint32_t pos[3] = {0, 17, Ma - 1};
    std::vector<uint16_t> Qr = rand_f16((size_t)H * 3 * D), Or((size_t)H * 3 * D);
    CHECK(orc_attention_rows(Qr.data(), Kx.data(), V.data(), Or.data(), pos, 3, H, Hkv, Ma, D, 0.125f, 0, 2) == 0);
    const uint32_t bad[1] = {Ma};
    CHECK(orc_attention_rows(Qr.data(), Kx.data(), V.data(), Or.data(), bad, 1, H, Hkv, Ma, D, 0.125f, 0, 2) == -4);
    std::vector<uint16_t> X = rand_f16((size_t)Ma * 128), w = rand_f16(128), Y((size_t)Ma * 128);
    CHECK(orc_rmsnorm(X.data(), w.data(), Y.data(), Ma, 128, 1e-5f, 1) == 0);
    CHECK(orc_rmsnorm(X.data(), w.data(), Y.data(), Ma, 128, 1e-5f, 2) == 0);
    CHECK(orc_rmsnorm(X.data(), w.data(), Y.data(), Ma, 128, 1e-5f, 3) == -3);
    CHECK(orc_rope(Q.data(), H, Ma, D, 10000.0f, 5, 0) == 0);
    CHECK(orc_rope(Q.data(), H, Ma, D, 500000.0f, 0, 1) == 0);
    CHECK(orc_rope(Q.data(), H, Ma, 63, 10000.0f, 0, 0) == -4);
    // layers: d_model 128, H 2 x D 64, MLP 256
    const uint32_t Ml = 9, dm = 128, Hl = 2, Dl = 64, Nm = 256;
    std::vector<uint16_t> Xl = rand_f16((size_t)Ml * dm), Xo((size_t)Ml * dm), na = rand_f16(dm), nf = rand_f16(dm);
    auto wq = rand_blocks(0, Hl * Dl, dm), wk = rand_blocks(0, Hl * Dl, dm), wv = rand_blocks(0, Hl * Dl, dm);
    auto wo = rand_blocks(0, dm, Hl * Dl), wg = rand_blocks(0, Nm, dm), wu = rand_blocks(0, Nm, dm);
    auto wd = rand_blocks(0, dm, Nm);
    CHECK(orc_layer(0, Xl.data(), wq.data(), wk.data(), wv.data(), wo.data(), wg.data(), wu.data(), wd.data(),
                    Xo.data(), Ml, dm, Hl, Dl, Nm, 0.125f, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                    2) == 0);
    auto wk1 = rand_blocks(0, Dl, dm), wv1 = rand_blocks(0, Dl, dm);
    CHECK(orc_layer_ex(0, Xl.data(), na.data(), wq.data(), wk1.data(), wv1.data(), wo.data(), nf.data(), wg.data(),
                       wu.data(), wd.data(), Xo.data(), Ml, dm, Hl, 1, Dl, Nm, 0.125f, 1, 1e-5f, 1, 10000.0f, 3, 0,
                       2) == 0);
    const uint32_t lpos[2] = {0, Ml - 1};
    std::vector<uint16_t> Xr((size_t)2 * dm);
    CHECK(orc_layer_ex_rows(0, Xl.data(), nullptr, wq.data(), wk.data(), wv.data(), wo.data(), nullptr, wg.data(),
                            wu.data(), wd.data(), Xr.data(), lpos, 2, Ml, dm, Hl, Hl, Dl, Nm, 0.125f, 1, 1e-5f, 0,
                            10000.0f, 0, 1, 2) == 0);
}

int main() {
    gguf_cases();
    registry_cases();
    host_cases();
    oracle_cases();
    printf("sanitize_host: ok\n");
    return 0;
}
