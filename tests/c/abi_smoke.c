/* A C caller of the drop-in boundary (include/m4_mlx_bridge.h, include/m4_gguf.h):
 * compiled with the host C compiler against the shipped library, exercising
 * the entry points that need no GPU (validation codes, expected sizes, the
 * registry, an uninitialized bridge, a GGUF buffer).  Exit status 0 = pass. */
#include <stdio.h>
#include <string.h>

#include "m4_gguf.h"
#include "m4_mlx_bridge.h"

#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); \
            return 1;                                              \
        }                                                          \
    } while (0)

static void le32(unsigned char* p, uint32_t v) { for (int i = 0; i < 4; i++) p[i] = (unsigned char)(v >> (8 * i)); }
static void le64(unsigned char* p, uint64_t v) { for (int i = 0; i < 8; i++) p[i] = (unsigned char)(v >> (8 * i)); }

int main(void) {
    /* core/bridge/m4_mlx_bridge.mm:58-75 */
    CHECK(m4_bridge_get_expected_weight_bytes(0, 4096, 4096) == 4096u / 32 * 4096 * 18);
    CHECK(m4_bridge_get_expected_weight_bytes(2, 4096, 4096) == 4096u / 256 * 4096 * 144);
    CHECK(m4_bridge_get_expected_weight_bytes(7, 4096, 4096) == 0);
    /* validation order and codes (m4_mlx_bridge.mm:201-230) */
    static char X[64 * 128 * 2], W[128 / 32 * 64 * 18], Y[64 * 64 * 2];
    CHECK(m4_bridge_validate_gemm(X, sizeof X, W, sizeof W, Y, sizeof Y, 0, 64, 128, 64) == 0);
    CHECK(m4_bridge_validate_gemm(NULL, sizeof X, W, sizeof W, Y, sizeof Y, 0, 64, 128, 64) == -2);
    CHECK(m4_bridge_validate_gemm(X, sizeof X, W, sizeof W, Y, sizeof Y, 6, 64, 128, 64) == -3);
    CHECK(m4_bridge_validate_gemm(X, sizeof X, W, sizeof W, Y, sizeof Y, 0, 64, 48, 64) == -4);
    CHECK(m4_bridge_validate_gemm(X, sizeof X, W, sizeof W - 1, Y, sizeof Y, 0, 64, 128, 64) == -2);
    /* registry (src/router/quant_registry.mm:60-172) */
    m4_quant_codec_info info;
    CHECK(m4_registry_get(2, &info) == 0);
    CHECK(strcmp(info.name, "Q4_K") == 0 && info.block_size == 256 && info.struct_size == 144);
    CHECK(strcmp(info.gemm_kernel_name, "quant_router_gemm_q4_k_64x64") == 0);
    CHECK(m4_registry_get_by_name("PRISM_Q2_0") == 7);
    CHECK(m4_registry_compute_weight_bytes(7, 4096 * 4096) == (uint64_t)4096 * 4096 / 128 * 34);
    /* a GGUF buffer: header, one u32 key, one tensor */
    static unsigned char g[256];
    size_t o = 0;
    memcpy(g, "GGUF", 4); o = 4;
    le32(g + o, 3); o += 4;
    le64(g + o, 1); o += 8;                 /* tensors */
    le64(g + o, 1); o += 8;                 /* metadata */
    le64(g + o, 9); o += 8; memcpy(g + o, "blk.count", 9); o += 9;
    le32(g + o, M4_GGUF_UINT32); o += 4; le32(g + o, 16); o += 4;
    le64(g + o, 1); o += 8; memcpy(g + o, "w", 1); o += 1;
    le32(g + o, 2); o += 4; le64(g + o, 128); o += 8; le64(g + o, 1); o += 8;
    le32(g + o, M4_GGML_PRISM_Q2_0); o += 4; le64(g + o, 0); o += 8;
    size_t data = (o + 31) / 32 * 32;
    CHECK(data + 34 <= sizeof g);
    g[data] = 0x00; g[data + 1] = 0x3c;     /* d = 1.0 */
    m4_gguf* f = m4_gguf_parse_buffer(g, data + 34);
    CHECK(f != NULL);
    CHECK(m4_gguf_version(f) == 3 && m4_gguf_tensor_count(f) == 1);
    CHECK(m4_gguf_get_uint32_metadata(f, "blk.count", 0) == 16);
    CHECK(m4_gguf_tensor_data_offset(f) == data);
    int fmt = -1; uint32_t K = 0, N = 0;
    unsigned char w[34];
    CHECK(m4_gguf_load_router_weights(f, "w", w, sizeof w, &fmt, &K, &N) == 34);
    CHECK(fmt == 7 && K == 128 && N == 1 && w[1] == 0x3c);
    m4_gguf_close(f);
    printf("abi_smoke: ok\n");
    return 0;
}
