/* m4_gguf.h -- GGUF ingestion for the quantization router (host code, C ABI).
 *
 * Replaces the reference's GGUFLoader (core/weights/gguf_loader.h:46-129,
 * core/weights/gguf_loader.mm:1-412): GGUF v2/v3 header, metadata table and
 * tensor table, zero-copy tensor access and the PrismML Q2_0 extraction.  It
 * adds the step the reference leaves to its callers: turning a checkpoint
 * tensor into the router's block layout, so GGUF weights feed the projection
 * kernels directly -- GGML Q4_0 / Q8_0 and PrismML Q2_0 blocks are already
 * router blocks; GGML-standard Q4_K is repacked into the router's own Q4_K
 * packing; MLX 4-bit g64 tensors (packed uint32 codes + fp16 scales/biases)
 * are repacked into MLX_4BIT 32-element blocks.  All repacks are lossless.
 *
 * Everything here runs on the host and needs no GPU.
 */
#ifndef M4_GGUF_H
#define M4_GGUF_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef M4_API
#define M4_API __attribute__((visibility("default")))
#endif

/* GGUF metadata value types (gguf_loader.h:12-26). */
enum {
    M4_GGUF_UINT8 = 0, M4_GGUF_INT8 = 1, M4_GGUF_UINT16 = 2, M4_GGUF_INT16 = 3, M4_GGUF_UINT32 = 4,
    M4_GGUF_INT32 = 5, M4_GGUF_FLOAT32 = 6, M4_GGUF_BOOL = 7, M4_GGUF_STRING = 8, M4_GGUF_ARRAY = 9,
    M4_GGUF_UINT64 = 10, M4_GGUF_INT64 = 11, M4_GGUF_FLOAT64 = 12
};

/* GGML tensor type ids the router ingests.  PrismML Q2_0 appears as 100 in
 * the reference's loader fixture (tests/test_gguf_loader.mm:82) and as 42 in
 * its Bonsai streamer (projects/bonsai/runtime/bonsai_weight_streamer.py:126);
 * both are accepted. */
enum {
    M4_GGML_F32 = 0, M4_GGML_F16 = 1, M4_GGML_Q4_0 = 2, M4_GGML_Q8_0 = 8, M4_GGML_Q4_K = 12,
    M4_GGML_PRISM_Q2_0 = 100, M4_GGML_PRISM_Q2_0_ALT = 42
};

typedef struct m4_gguf m4_gguf;

/* GGUFTensorInfo (gguf_loader.h:38-45); dims[0] = ne0 (K, the contiguous
 * axis), dims[1] = ne1 (N).  At most 4 dims are reported. */
typedef struct {
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;
    uint64_t offset;      /* relative to the tensor data offset */
} m4_gguf_tensor_info;

/* GGUFLoader::open (gguf_loader.mm:150-186): mmap + parse; NULL on failure. */
M4_API m4_gguf* m4_gguf_open(const char* path);
/* GGUFLoader::parse_from_buffer (:188-203): parses `data` in place; the
 * caller keeps it alive until m4_gguf_close.  NULL on failure. */
M4_API m4_gguf* m4_gguf_parse_buffer(const void* data, size_t size);
M4_API void m4_gguf_close(m4_gguf* g);

M4_API uint32_t m4_gguf_version(const m4_gguf* g);
M4_API uint64_t m4_gguf_tensor_count(const m4_gguf* g);
M4_API uint64_t m4_gguf_metadata_count(const m4_gguf* g);
M4_API uint32_t m4_gguf_alignment(const m4_gguf* g);
M4_API uint64_t m4_gguf_tensor_data_offset(const m4_gguf* g);
M4_API size_t m4_gguf_file_size(const m4_gguf* g);

/* Metadata access (gguf_loader.h:72-77).  type: -1 if absent.  String:
 * returns the length (writing up to cap - 1 bytes + NUL into out when out is
 * not NULL), or -1 if absent or not a string. */
M4_API bool m4_gguf_has_metadata(const m4_gguf* g, const char* key);
M4_API int m4_gguf_metadata_type(const m4_gguf* g, const char* key);
M4_API int64_t m4_gguf_get_string_metadata(const m4_gguf* g, const char* key, char* out, size_t cap);
M4_API uint32_t m4_gguf_get_uint32_metadata(const m4_gguf* g, const char* key, uint32_t def);
M4_API uint64_t m4_gguf_get_uint64_metadata(const m4_gguf* g, const char* key, uint64_t def);
/* Numeric value of a scalar entry as double (ints, floats, bools); def if
 * absent or not scalar numeric.  Array length: -1 if absent / not an array. */
M4_API double m4_gguf_get_number_metadata(const m4_gguf* g, const char* key, double def);
M4_API int64_t m4_gguf_get_array_length(const m4_gguf* g, const char* key);

/* Tensor access (gguf_loader.h:79-85): names in file order. */
M4_API bool m4_gguf_has_tensor(const m4_gguf* g, const char* name);
M4_API int m4_gguf_get_tensor_info(const m4_gguf* g, const char* name, m4_gguf_tensor_info* out);
M4_API const char* m4_gguf_tensor_name(const m4_gguf* g, uint64_t index);
M4_API const void* m4_gguf_get_tensor_raw_data(const m4_gguf* g, const char* name);

/* GGUFLoader::extract_q2_0_tensor (gguf_loader.mm:349-409): copies the
 * tensor's 34-byte PrismML Q2_0 blocks into dst (cap bytes) and reports
 * K = dims[0], N = dims[1] (1 for a vector).  Returns the block count, or -1
 * (missing tensor, no dims, element count not a multiple of 128, file bounds,
 * or dst too small). */
M4_API int64_t m4_gguf_extract_q2_0_tensor(const m4_gguf* g, const char* name, void* dst, size_t cap,
                                           uint64_t* out_k, uint64_t* out_n);

/* Router weights of tensor `name`: the bytes the projection entry points take
 * for W [N, K] (N = dims[1], K = dims[0]) in *format (0 Q4_0, 2 Q4_K,
 * 6 Q8_0, 7 PRISM_Q2_0).  With dst NULL only reports the size.  Returns the
 * byte count, -1 (missing tensor / bounds), -3 (tensor type without a router
 * format), -4 (K not a whole number of blocks) or -2 (dst too small). */
M4_API int64_t m4_gguf_load_router_weights(const m4_gguf* g, const char* name, void* dst, size_t cap,
                                           int* format, uint32_t* K, uint32_t* N);

/* GGML-standard Q4_K super-blocks (ggml block_q4_K: d, dmin, scales[12] in
 * get_scale_min_k4 packing, qs[128] with 32-byte chunks holding elements
 * 64 c + l in the low and 64 c + 32 + l in the high nibbles) -> the router's
 * Q4_K blocks (quant_router.h:49-55; cpu_gold_reference.h:116-144).  Same
 * weights exactly.  src and dst may not overlap.  Returns 0. */
M4_API int m4_repack_ggml_q4_k(const void* src, size_t num_blocks, void* dst);

/* MLX 4-bit affine, group 64: wq uint32 [N, K / 8] (code j of a word at bits
 * 4 j, element 8 w + j), scales and biases fp16 [N, K / 64]; w = scale q + bias.
 * -> router MLX_4BIT blocks [N, K / 32] x 20 bytes (each group becomes two
 * blocks with the same scale and bias).  Returns 0, or -4 if K % 64. */
M4_API int m4_repack_mlx_g64(const void* wq, const void* scales, const void* biases, uint32_t N, uint32_t K,
                             void* dst);

#ifdef __cplusplus
}
#endif

#endif /* M4_GGUF_H */
