/*
 * m4_mlx_bridge.h -- C-ABI of the MI355X quantization-router prefill path.
 *
 * Drop-in for the reference's core/bridge/m4_mlx_bridge.h:23-106: the same
 * eight entry points with the same argument meaning, return values and
 * validation order, exported from libm4_bridge.so.  Pointers are DEVICE
 * pointers (hipMalloc / torch-ROCm data_ptr()); host pointers are accepted
 * too and staged through device memory (slower, PCIe-bound).  Kernels run
 * on the bridge stream (m4_bridge_set_stream) asynchronously;
 * m4_bridge_synchronize() waits for everything issued so far.
 *
 * Error codes (checked in this order, before any device work,
 * core/bridge/m4_mlx_bridge.mm:201-230):
 *   -1 bridge not initialized
 *   -2 null pointer, odd (non-2-byte-aligned) X or Y, or a buffer too small
 *   -3 invalid format (the projection entry points accept ids 0..5)
 *   -4 invalid dimension: M, K or N zero; K % 32; K % 256 for formats 2, 4, 5
 *   -5 device staging allocation failed
 *   -6 kernel launch / device failure
 *
 * The entry points below the first block have no single counterpart in the
 * reference's C-ABI; each names the reference routine it replaces.
 */
#ifndef M4_MLX_BRIDGE_H
#define M4_MLX_BRIDGE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define M4_API __attribute__((visibility("default")))
#else
#define M4_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference C-ABI (core/bridge/m4_mlx_bridge.h) ---------------------- */

/* m4_mlx_bridge.h:23 -- selects the HIP device, creates the bridge stream.
 * The path argument is accepted for compatibility and ignored (kernels are
 * compiled into the library). */
M4_API bool m4_bridge_init(const char* metallib_path);

/* m4_mlx_bridge.h:33 -- minimum W bytes for format 0..5, else 0. */
M4_API size_t m4_bridge_get_expected_weight_bytes(int format, uint32_t K, uint32_t N);

/* m4_mlx_bridge.h:57 -- Y[M,N] (fp16) = X[M,K] (fp16) . W^T, W packed [N, K]. */
M4_API int m4_bridge_dispatch_gemm(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes, void* Y_ptr,
                            size_t Y_bytes, int format, uint32_t M, uint32_t K, uint32_t N);

/* m4_mlx_bridge.h:79 -- GEMM with M = 1 (m4_mlx_bridge.mm:293-302). */
M4_API int m4_bridge_dispatch_gemv(void* x_ptr, size_t x_bytes, void* W_ptr, size_t W_bytes, void* y_ptr,
                            size_t y_bytes, int format, uint32_t K, uint32_t N);

/* m4_mlx_bridge.h:90 -- waits for all work issued on the bridge stream. */
M4_API void m4_bridge_synchronize(void);

/* m4_mlx_bridge.h:96 -- process footprint in MB: host resident set plus the
 * device memory the bridge itself holds. */
M4_API double m4_bridge_get_uma_footprint_mb(void);

/* m4_mlx_bridge.h:101 */
M4_API bool m4_bridge_is_initialized(void);

/* m4_mlx_bridge.h:106 -- waits, releases staging memory and the stream. */
M4_API void m4_bridge_shutdown(void);

/* ---- extensions: same router, other reference routines ------------------ */

/* Validation only: the code m4_bridge_dispatch_gemm would return for these
 * arguments on an initialized bridge (0 if it would launch), computed without
 * touching a device (m4_mlx_bridge.mm:204-230). */
M4_API int m4_bridge_validate_gemm(const void* X_ptr, size_t X_bytes, const void* W_ptr, size_t W_bytes,
                            const void* Y_ptr, size_t Y_bytes, int format, uint32_t M, uint32_t K,
                            uint32_t N);

/* Projection for every format with a kernel: formats 0..5 as
 * m4_bridge_dispatch_gemm, plus PRISM_Q2_0 (7; K % 128 == 0) and Q8_0 weights
 * (6).  Replaces the registry's kernels reached by name,
 * quant_router_gemm_<fmt>_64x64 (quant_router_kernels.metal:588-750,
 * prism_q2_0 at :726; names from src/router/quant_registry.mm:60-172 --
 * quant_router_gemm_q8_0_64x64 is named there but has no Metal kernel).
 * Same validation order and codes as dispatch_gemm with the wider format set. */
M4_API int m4_bridge_dispatch_router_gemm(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes, void* Y_ptr,
                                   size_t Y_bytes, int format, uint32_t M, uint32_t K, uint32_t N);

/* Direct-head projection: Y is [H, M, D] with N = H * D; replaces
 * quant_router_head_gemm_<fmt>_64x64 (quant_router_kernels.metal:754-927,
 * index map :570-574).  Same validation as dispatch_router_gemm with N = H * D
 * (formats 0..7). */
M4_API int m4_bridge_dispatch_head_gemm(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes, void* Y_ptr,
                                 size_t Y_bytes, int format, uint32_t M, uint32_t H, uint32_t D,
                                 uint32_t K);

/* A router kernel by its Metal pipeline name, with that kernel's buffer and
 * constant slots: A = X (buffer 0), B = W (1), C = Y (2), and dims = the
 * constants from slot 3 on -- {M, N, K} for quant_router_gemm_<fmt>_64x64
 * (quant_router_kernels.metal:588-750) and {M, H, D, K} for
 * quant_router_head_gemm_<fmt>_64x64 (:754-927); kernel names as listed by the
 * registry (src/router/quant_registry.mm:60-172).  The vector-ALU ternary
 * kernels quant_router_gemm_ternary_1_58_vec (:934-1064) and
 * quant_router_head_gemm_ternary_1_58_vec (:1067-1201) compute the same
 * projection and run the matrix-core path here.  Returns -3 for an unknown
 * name, -4 when ndims does not match the kernel's constant slots, otherwise
 * what dispatch_router_gemm / dispatch_head_gemm return. */
M4_API int m4_bridge_dispatch_router_kernel(const char* kernel_name, void* X_ptr, size_t X_bytes, void* W_ptr,
                                            size_t W_bytes, void* Y_ptr, size_t Y_bytes, const uint32_t* dims,
                                            uint32_t ndims);

/* Projection with a fused residual: Y = fp16(X . W^T + R), R fp16 [M, N];
 * replaces a GEMM followed by vector_add_residual (unified_kernels.metal:
 * 78-88; unified_prefill_engine.mm:183-186).  Y may alias R. */
M4_API int m4_bridge_dispatch_gemm_residual(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes,
                                     void* R_ptr, size_t R_bytes, void* Y_ptr, size_t Y_bytes,
                                     int format, uint32_t M, uint32_t K, uint32_t N);

/* Fused dual-projection SwiGLU: Out[M, N_mlp] = silu(X . Wg^T) * (X . Wu^T);
 * replaces swiglu_mma_dual_simd (brick3_swiglu_kernels.metal:428-698), which
 * takes Q4_0 only; any format with kernels (0..7) is accepted here. */
M4_API int m4_bridge_dispatch_swiglu(void* X_ptr, size_t X_bytes, void* Wg_ptr, size_t Wg_bytes, void* Wu_ptr,
                              size_t Wu_bytes, void* Out_ptr, size_t Out_bytes, int format, uint32_t M,
                              uint32_t N_mlp, uint32_t K);

/* Q8_0 quantization of num_blocks groups of 32 fp16 values into 34-byte
 * blocks; replaces quantize_kv_to_q8_0 (unified_kernels.metal:118-145). */
M4_API int m4_bridge_quantize_kv_q8_0(void* src_ptr, size_t src_bytes, void* dst_ptr, size_t dst_bytes,
                               uint64_t num_blocks);

/* Causal flash attention over a Q8_0 KV cache; replaces
 * flash_attn_mma_64x64_q8_0_d64/_d128 (brick4_attn_kernels.metal:868-911).
 * Q fp16 [H, M, D]; K_q8, V_q8 Q8_0 blocks over [H, M, D]; D in {64, 128}.
 * O fp16 [H, M, D] (o_token_major = 0) or [M, H * D] (o_token_major = 1). */
M4_API int m4_bridge_dispatch_flash_attn_q8_0(void* Q_ptr, size_t Q_bytes, void* Kq_ptr, size_t Kq_bytes,
                                       void* Vq_ptr, size_t Vq_bytes, void* O_ptr, size_t O_bytes,
                                       uint32_t H, uint32_t M, uint32_t D, float scale,
                                       int o_token_major);

/* One prefill layer (no norm, no RoPE), composed as the reference's
 * TransformerLayerCoordinator::forward (models/transformer_layer.mm:75-218)
 * with the Q8_0 KV cache of unified_prefill_engine.mm:554-572:
 *   Q,K,V head GEMMs -> Q8_0(K,V) -> flash attention -> O-proj + residual ->
 *   fused SwiGLU -> down-proj + residual.
 * X, X_out fp16 [M, d_model]; Wq/Wk/Wv [H*D, d_model], Wo [d_model, H*D],
 * Wg/Wu [N_mlp, d_model], Wd [d_model, N_mlp], all in `format`.  Scratch is
 * held by the bridge.  X_out must not alias X. */
M4_API int m4_bridge_prefill_layer(void* X_ptr, void* Wq, void* Wk, void* Wv, void* Wo, void* Wg, void* Wu,
                            void* Wd, void* X_out, int format, uint32_t M, uint32_t d_model, uint32_t H,
                            uint32_t D, uint32_t N_mlp, float attn_scale);

/* Grouped-query variant: K/V carry Hkv heads ([Hkv, M, D] Q8_0 blocks) and
 * query head h reads KV head h / (H / Hkv) (H % Hkv == 0), as the MLX block
 * passes them to scaled_dot_product_attention (src/engine/model.py:234-236).
 * Hkv == H is m4_bridge_dispatch_flash_attn_q8_0. */
M4_API int m4_bridge_dispatch_flash_attn_q8_0_gqa(void* Q_ptr, size_t Q_bytes, void* Kq_ptr, size_t Kq_bytes,
                                           void* Vq_ptr, size_t Vq_bytes, void* O_ptr, size_t O_bytes,
                                           uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D, float scale,
                                           int o_token_major);

/* RMSNorm of the MLX block (src/engine/model.py:17-48) over rows of X [M, D]
 * (D % 8 == 0): Y = fp16(fp16(x / sqrt(mean(x^2) + eps)) * w) for norm_type 1
 * ("rmsnorm"), with fp16(1 + w) in place of w for norm_type 2
 * ("gemma_add_one").  W fp16 [D].  Codes: -1, -2 (null / short buffers),
 * -3 (norm_type), -4 (dims), -5, -6 as dispatch_gemm. */
M4_API int m4_bridge_rmsnorm(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes, void* Y_ptr,
                      size_t Y_bytes, uint32_t M, uint32_t D, float eps, int norm_type);

/* Rotary position embedding in place on T [H, M, D] (D % 16 == 0): nn.RoPE
 * (dims = D, traditional, base = theta) applied at positions offset + m
 * (src/engine/model.py:112-116, :215-226).  Pairs (i, i + D/2), or (2i, 2i + 1)
 * when traditional, rotate by (offset + m) theta^(-2i/D). */
M4_API int m4_bridge_rope(void* T_ptr, size_t T_bytes, uint32_t H, uint32_t M, uint32_t D, float theta,
                   uint32_t offset, int traditional);

/* The MLX transformer block (src/engine/model.py:181-265) on the router's
 * kernels: RMSNorm(X, w_attn) -> Q [Hq], K, V [Hkv] head GEMMs -> RoPE(Q, K)
 * -> Q8_0(K, V) -> grouped-query flash attention -> O-proj + residual ->
 * RMSNorm(w_ffn) -> fused SwiGLU -> down-proj + residual.  w_attn / w_ffn
 * fp16 [d_model] or NULL (no norm); rope = 0 skips RoPE.  Wq [Hq*D, d_model],
 * Wk/Wv [Hkv*D, d_model], Wo [d_model, Hq*D], Wg/Wu [N_mlp, d_model],
 * Wd [d_model, N_mlp].  Device pointers, 16-byte aligned; X_out must not
 * alias X.  Hkv == Hq, no norms, no RoPE is m4_bridge_prefill_layer. */
M4_API int m4_bridge_prefill_layer_ex(void* X_ptr, void* w_attn, void* Wq, void* Wk, void* Wv, void* Wo,
                               void* w_ffn, void* Wg, void* Wu, void* Wd, void* X_out, int format,
                               uint32_t M, uint32_t d_model, uint32_t Hq, uint32_t Hkv, uint32_t D,
                               uint32_t N_mlp, float attn_scale, int norm_type, float norm_eps, int rope,
                               float rope_theta, uint32_t rope_offset, int rope_traditional);

/* m4_bridge_prefill_layer_ex that also hands back the layer's Q8_0 KV cache
 * (the d_K_q8 / d_V_q8 buffers of unified_prefill_engine.mm:548-572): Kq_out
 * and Vq_out, device memory of Hkv * M * D / 32 * 34 bytes each, receive the
 * Q8_0 blocks of K and V ([Hkv, M, D], 32 consecutive d per 34-byte block,
 * K after RoPE).  Both NULL: m4_bridge_prefill_layer_ex; only one: -2. */
M4_API int m4_bridge_prefill_layer_ex_kv(void* X_ptr, void* w_attn, void* Wq, void* Wk, void* Wv, void* Wo,
                                  void* w_ffn, void* Wg, void* Wu, void* Wd, void* X_out, void* Kq_out,
                                  void* Vq_out, int format, uint32_t M, uint32_t d_model, uint32_t Hq, uint32_t Hkv,
                                  uint32_t D, uint32_t N_mlp, float attn_scale, int norm_type, float norm_eps,
                                  int rope, float rope_theta, uint32_t rope_offset, int rope_traditional);

/* Dequantize W [N, K] to fp16 [N, K] with the kernels' own decoders (the
 * registry's dequantize hook, src/router/quant_registry.h:24). Formats 0..7. */
M4_API int m4_bridge_dequantize(void* W_ptr, size_t W_bytes, void* out_ptr, size_t out_bytes, int format,
                         uint32_t K, uint32_t N);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): m4_bridge_dispatch_gemm's projection with the same
 * arguments, validation and results, but its split-K partials live in a
 * fixed 32 MiB device scratch array of the library (one per GPU, held until
 * the process ends) and no device memory is allocated or freed.  X, W and Y
 * must be device memory (X and W 16-byte aligned): -2 otherwise, since host
 * or misaligned buffers would need staging copies.  -4 when the shape needs
 * more split-K partials than the scratch holds (ksplit * M * N <= 8 Mi
 * floats: every tiled launch fits; small-M launches with long K and wide N,
 * e.g. M = 48, K = 16384, N = 12288, do not).  Calls on one GPU share the scratch: calls
 * that overlap in time (other streams, other threads' streams) race. */
M4_API int m4_bridge_dispatch_gemm_noalloc(void* X_ptr, size_t X_bytes, void* W_ptr, size_t W_bytes, void* Y_ptr,
                                           size_t Y_bytes, int format, uint32_t M, uint32_t K, uint32_t N);

/* Run subsequent work on `stream` (a hipStream_t, e.g. torch's current
 * stream); NULL restores the bridge's own stream.  Returns 0 or -1. */
M4_API int m4_bridge_set_stream(void* stream);
/* The hipStream_t work is issued on. */
M4_API void* m4_bridge_get_stream(void);
/* Text of the last error this thread's bridge calls saw ("" if none); per
 * thread, like errno, so a caller reads the message of its own failed call. */
M4_API const char* m4_bridge_last_error(void);

/* ---- roofline probes (quant_router_kernels.metal:71-104, timed as in
 *      bench_universal_router.mm:645-717) ------------------------------- */

/* probe_memory_bandwidth: HBM GB/s of a read-only stream over `bytes` (> the
 * 256 MB Infinity Cache to measure HBM) and of the reference's dst = src + 1
 * copy (bytes read + written), best of `reps` timed runs after one warmup.
 * Allocates its own buffers; runs on the null stream.  0, -2, -4 or -6. */
M4_API int m4_probe_hbm_bandwidth(size_t bytes, int reps, double* read_gbs, double* copy_gbs);
/* probe_fma_roofline, on the matrix pipe: dense fp16 TFLOP/s of back-to-back
 * v_mfma_f32_32x32x16_f16 on every SIMD (`iters` rounds of 4 independent
 * chains per wave), best of `reps`, and the average shader clock (GHz) the
 * waves saw (shader-cycle counter over the 100 MHz real-time counter).
 * `iters` >= 64 and a multiple of 4.  0, -2, -4 or -6. */
M4_API int m4_probe_mfma_f16(uint32_t iters, int reps, double* tflops, double* clock_ghz);
/* The same with random fp16 operands (four A and four B fragments per lane,
 * values in [-1, 1)): the matrix pipe draws more power when more operand bits
 * toggle, and the part lowers its clock, so this is the dense ceiling real
 * activations and weights can reach.  No counterpart in the reference (its
 * FMA probe is operand-independent).  `iters` a multiple of 4.  0, -2, -4, -6. */
M4_API int m4_probe_mfma_f16_random(uint32_t iters, int reps, double* tflops, double* clock_ghz);

/* ---- format registry (src/router/quant_registry.h:14-65) ---------------- */

typedef struct {
    int format;
    const char* name;
    const char* description;
    uint32_t block_size;
    uint64_t struct_size;
    double bits_per_weight;
    const char* gemm_kernel_name;
    const char* head_gemm_kernel_name;
} m4_quant_codec_info;

/* QuantRegistry::get -- 0 and *out filled, or -3 if unknown. */
M4_API int m4_registry_get(int format, m4_quant_codec_info* out);
/* QuantRegistry::get_by_name -- format id or -3. */
M4_API int m4_registry_get_by_name(const char* name);
/* QuantRegistry::available_formats -- count; ids written to out[0..cap). */
M4_API int m4_registry_available_formats(int* out, int cap);
/* QuantRegistry::compute_weight_bytes -- 0 for an unknown format. */
M4_API uint64_t m4_registry_compute_weight_bytes(int format, uint64_t num_elements);
/* QuantRegistry::has_format */
M4_API bool m4_registry_has_format(int format);
/* QuantRegistry::register_codec (e.g. QUANT_CUSTOM = 99); strings are copied. */
M4_API int m4_registry_register_codec(const m4_quant_codec_info* info);

#ifdef __cplusplus
}
#endif

#endif /* M4_MLX_BRIDGE_H */
