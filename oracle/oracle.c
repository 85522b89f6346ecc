/*
 * oracle.c -- CPU restatement of m4-prefill-engine's double-precision
 * verification path for the quantization-router prefill path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker.  The product (libm4_bridge.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates.  The reference's
 * gold code is ObjC++ with Grand Central Dispatch blocks and `__fp16`
 * (tests/e2e/cpu_gold_reference.h:7,27), which cannot be compiled on Linux;
 * this file restates the same double arithmetic in C with POSIX threads in
 * place of dispatch_apply, and explicit IEEE binary16 conversions in place of
 * the `(__fp16)` casts:
 *   - `(double)h` of an fp16 value is exact (f16_to_f64);
 *   - `(__fp16)x` of a double is ONE round-to-nearest-even rounding
 *     (f64_to_f16), as clang's double->half conversion on arm64.
 *
 * Byte layouts (quant_router.h:35-96), all little-endian:
 *   Q4_0     18 B / 32: f16 d | u8 qs[16]
 *   MLX_4BIT 20 B / 32: f16 d | f16 bias | u8 qs[16]
 *   Q4_K    144 B / 256: f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
 *   TERNARY  12 B / 32: f16 d | f16 pad | u32 qs[2]
 *   VAR_RATE 160 B / 256: f16 d | f16 bias | u8 scales[8] | u8 biases[8] |
 *                        u8 modes[8] | u8 pad[4] | u8 qs[128]
 *   EXL3    144 B / 256: f16 d | f16 bias | u8 scales[8] | u8 residuals[8] |
 *                        i8 codebook[16] | u8 pad[12] | u8 qs[96]
 *   Q8_0     34 B / 32: f16 d | i8 qs[32]
 *   PRISM    34 B / 128: f16 d | u8 qs[32]
 *   MLX_G64  36 B / 64: f16 scale | f16 bias | u32 qs[8]  (MLX's own layout)
 *
 * Parity pins for each function are listed in tests/test_oracle.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

/* Allocation failure: row workers skip their row and raise this flag, which
 * the exported functions that return a status report as -5; the others stop
 * with a message (they have no status to return). */
static int g_alloc_failed = 0;
static void* row_alloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) __atomic_store_n(&g_alloc_failed, 1, __ATOMIC_RELAXED);
    return p;
}
static void* must_alloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory allocating %zu bytes\n", n);
        abort();
    }
    return p;
}
static int take_alloc_status(void) { return __atomic_exchange_n(&g_alloc_failed, 0, __ATOMIC_RELAXED) ? -5 : 0; }

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary64                                               */
/* ------------------------------------------------------------------------ */

EXPORT double orc_f16_to_f64(uint16_t h) {
    int s = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), e - 25);
    return s ? -v : v;
}

/* Round-to-nearest-even double -> binary16 (single rounding). */
EXPORT uint16_t orc_f64_to_f16(double x) {
    uint16_t sign = signbit(x) ? 0x8000 : 0;
    if (isnan(x)) return 0x7e00;
    double a = fabs(x);
    if (a == 0.0) return sign;
    /* largest finite half is 65504; values >= 65520 round to inf */
    if (a >= 65520.0) return sign | 0x7c00;
    int e;
    frexp(a, &e);              /* a = f * 2^e, f in [0.5,1) */
    int ex = e - 1;            /* a in [2^ex, 2^(ex+1)) */
    if (ex < -14) ex = -14;    /* subnormal range: fixed quantum 2^-24 */
    double q = ldexp(a, 10 - ex);   /* scaled so the kept bits are the integer part */
    double fl = floor(q);
    double rem = q - fl;       /* exact: q has <= 53 bits */
    uint64_t mant = (uint64_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (mant & 1))) mant++;
    /* mant is the significand incl. implicit bit, scaled at 2^(ex-10) */
    if (mant == 0x800) { mant = 0x400; ex++; }
    if (ex > 15) return sign | 0x7c00;
    if (mant < 0x400) return sign | (uint16_t)mant;   /* subnormal (ex == -14) */
    return sign | (uint16_t)(((ex + 15) << 10) | (mant & 0x3ff));
}

EXPORT void orc_f64_to_f16_array(const double* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f64_to_f16(x[i]);
}

EXPORT void orc_f16_to_f64_array(const uint16_t* x, double* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f64(x[i]);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline double hf(const uint8_t* p) { return orc_f16_to_f64(rd16(p)); }

/* float (binary32) helpers used where the reference computes in float */
static inline float f16_to_f32(uint16_t h) { return (float)orc_f16_to_f64(h); }
static inline uint16_t f32_to_f16(float x) { return orc_f64_to_f16((double)x); }

/* ------------------------------------------------------------------------ */
/* Format table (quant_router.h:110-136; core/bridge/m4_mlx_bridge.mm:58-75) */
/* ------------------------------------------------------------------------ */

enum { F_Q4_0 = 0, F_MLX = 1, F_Q4_K = 2, F_TERN = 3, F_VAR = 4, F_EXL3 = 5, F_Q8_0 = 6, F_PRISM = 7, F_G64 = 8 };
#define F_LAST F_G64

static const uint32_t kBlockElems[9] = {32, 32, 256, 32, 256, 256, 32, 128, 64};
static const uint32_t kBlockBytes[9] = {18, 20, 144, 12, 160, 144, 34, 34, 36};

EXPORT uint32_t orc_block_elems(int f) { return (f >= 0 && f <= F_LAST) ? kBlockElems[f] : 0; }
EXPORT uint32_t orc_block_bytes(int f) { return (f >= 0 && f <= F_LAST) ? kBlockBytes[f] : 0; }

/*
 * Exact weights of ONE block, in element order, as doubles, plus the order in
 * which the reference's gold loop visits (element, activation index) pairs.
 *
 * Each decoder restates the reference's CPU gold formula; the value written to
 * w[j] is the exact double the reference multiplies a_row[k0 + j] with.
 */

/* Q4_0: cpu_gold_reference.h:33-41 -> w = (q-8)*d; byte i low nibble is element
 * i, high nibble element i+16. */
static void dec_q4_0(const uint8_t* b, double w[32]) {
    double d = hf(b);
    for (int i = 0; i < 16; i++) {
        uint8_t v = b[2 + i];
        w[i] = (double)((int)(v & 0x0f) - 8) * d;
        w[i + 16] = (double)((int)(v >> 4) - 8) * d;
    }
}

/* MLX_4BIT: cpu_gold_reference.h:73-84 -> w = q*d + bias. */
static void dec_mlx(const uint8_t* b, double w[32]) {
    double d = hf(b), bias = hf(b + 2);
    for (int i = 0; i < 16; i++) {
        uint8_t v = b[4 + i];
        w[i] = (double)(v & 0x0f) * d + bias;
        w[i + 16] = (double)(v >> 4) * d + bias;
    }
}

/* Q4_K: cpu_gold_reference.h:116-144 (the reference's own 6-bit packing). */
static void dec_q4_k(const uint8_t* b, double w[256]) {
    double d = hf(b), dmin = hf(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* qs = b + 16;
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 4; j++) {
        sc[j] = scales[j] & 0x3f;
        sc[j + 4] = scales[j + 4] & 0x3f;
        mn[j] = (scales[j + 8] & 0x0f) | ((scales[j] >> 6) << 4);
        mn[j + 4] = ((scales[j + 8] >> 4) & 0x0f) | ((scales[j + 4] >> 6) << 4);
    }
    for (int s = 0; s < 8; s++) {
        double dsub = d * (double)sc[s];
        double msub = dmin * (double)mn[s];
        for (int i = 0; i < 16; i++) {
            uint8_t v = qs[s * 16 + i];
            w[s * 32 + i] = (double)(v & 0x0f) * dsub - msub;
            w[s * 32 + i + 16] = (double)(v >> 4) * dsub - msub;
        }
    }
}

/* TERNARY_1_58: cpu_gold_reference.h:176-187 -> w = (c-1)*d, 2-bit codes
 * LSB-first; qs[0] holds elements 0..15, qs[1] elements 16..31.  Code 3 gives
 * +2*d in the CPU gold (the reference's Metal kernel clamps it to 0,
 * quant_router_kernels.metal:253); this oracle follows the CPU gold. */
static void dec_tern(const uint8_t* b, double w[32]) {
    double d = hf(b);
    uint32_t q0 = rd32(b + 4), q1 = rd32(b + 8);
    for (int j = 0; j < 16; j++) {
        w[j] = (double)((int)((q0 >> (2 * j)) & 3) - 1) * d;
        w[16 + j] = (double)((int)((q1 >> (2 * j)) & 3) - 1) * d;
    }
}

/* VAR_RATE_AFFINE: cpu_gold_reference.h:212-323.  Returns weights in
 * ACTIVATION order (the permutation is applied), i.e. w[k] multiplies a[k]. */
static void dec_var(const uint8_t* b, double w[256]) {
    static const uint32_t off[8] = {0, 12, 24, 40, 56, 72, 88, 108};
    double d = hf(b), bias = hf(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* biases = b + 12;
    const uint8_t* modes = b + 20;
    const uint8_t* qs = b + 32;
    for (int s = 0; s < 8; s++) {
        double sub_scale = d * (double)scales[s] * 0.0625;
        double sub_bias = bias + d * ((double)biases[s] - 128.0) * 0.0625;
        uint8_t bits = modes[s] & 7, perm = (modes[s] >> 3) & 3;
        const uint8_t* p = qs + off[s];
        double u[32];
        if (bits == 3) {
            for (int g = 0; g < 4; g++) {
                uint8_t b0 = p[g * 3], b1 = p[g * 3 + 1], b2 = p[g * 3 + 2];
                uint8_t q[8] = {(uint8_t)(b0 & 7), (uint8_t)((b0 >> 3) & 7),
                                (uint8_t)(((b0 >> 6) | (b1 << 2)) & 7), (uint8_t)((b1 >> 1) & 7),
                                (uint8_t)((b1 >> 4) & 7), (uint8_t)(((b1 >> 7) | (b2 << 1)) & 7),
                                (uint8_t)((b2 >> 2) & 7), (uint8_t)((b2 >> 5) & 7)};
                for (int i = 0; i < 8; i++) u[g * 8 + i] = ((double)q[i] - 4.0) * sub_scale + sub_bias;
            }
        } else if (bits == 5) {
            for (int g = 0; g < 4; g++) {
                const uint8_t* c = p + g * 5;
                uint8_t q[8] = {(uint8_t)(c[0] & 31), (uint8_t)(((c[0] >> 5) | (c[1] << 3)) & 31),
                                (uint8_t)((c[1] >> 2) & 31), (uint8_t)(((c[1] >> 7) | (c[2] << 1)) & 31),
                                (uint8_t)(((c[2] >> 4) | (c[3] << 4)) & 31), (uint8_t)((c[3] >> 1) & 31),
                                (uint8_t)(((c[3] >> 6) | (c[4] << 2)) & 31), (uint8_t)((c[4] >> 3) & 31)};
                for (int i = 0; i < 8; i++) u[g * 8 + i] = ((double)q[i] - 16.0) * sub_scale + sub_bias;
            }
        } else {
            for (int i = 0; i < 16; i++) {
                u[i] = ((double)(p[i] & 15) - 8.0) * sub_scale + sub_bias;
                u[16 + i] = ((double)(p[i] >> 4) - 8.0) * sub_scale + sub_bias;
            }
        }
        for (int j = 0; j < 32; j++) {
            int dst = j;
            if (perm == 1) dst = ((j & 1) << 4) | (j >> 1);
            else if (perm == 2) dst = 31 - j;
            w[s * 32 + dst] = u[j];
        }
    }
}

/* EXL3: cpu_gold_reference.h:345-392. */
static void dec_exl3(const uint8_t* b, double w[256]) {
    double d = hf(b), bias = hf(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* res = b + 12;
    const int8_t* cb = (const int8_t*)(b + 20);
    const uint8_t* qs = b + 48;
    for (int s = 0; s < 8; s++) {
        double sub_scale = d * (double)scales[s] * 0.015625;
        double sub_res = d * ((double)res[s] - 128.0) * 0.0078125;
        const uint8_t* p = qs + s * 12;
        for (int g = 0; g < 4; g++) {
            uint8_t b0 = p[g * 3], b1 = p[g * 3 + 1], b2 = p[g * 3 + 2];
            uint8_t q[8] = {(uint8_t)(b0 & 7), (uint8_t)((b0 >> 3) & 7),
                            (uint8_t)(((b0 >> 6) | (b1 << 2)) & 7), (uint8_t)((b1 >> 1) & 7),
                            (uint8_t)((b1 >> 4) & 7), (uint8_t)(((b1 >> 7) | (b2 << 1)) & 7),
                            (uint8_t)((b2 >> 2) & 7), (uint8_t)((b2 >> 5) & 7)};
            for (int i = 0; i < 8; i++)
                w[s * 32 + g * 8 + i] = bias + sub_scale * (double)cb[q[i]] + sub_res * (double)cb[q[i] + 8];
        }
    }
}

/* Q8_0 weights: w = q*d (the registry names a Q8_0 GEMM, quant_registry.mm:153;
 * the block is the KV-cache block of brick4_attn_bench.mm:57-65). */
static void dec_q8_0(const uint8_t* b, double w[32]) {
    double d = hf(b);
    for (int i = 0; i < 32; i++) w[i] = (double)(int8_t)b[2 + i] * d;
}

/* PRISM_Q2_0: cpu_gold_reference.h:418-430 -> w = (c-1)*d, 4 codes per byte
 * LSB-first, element byte*4+j. */
static void dec_prism(const uint8_t* b, double w[128]) {
    double d = hf(b);
    for (int i = 0; i < 32; i++)
        for (int j = 0; j < 4; j++) w[i * 4 + j] = (double)((int)((b[2 + i] >> (2 * j)) & 3) - 1) * d;
}

/* MLX_4BIT_G64 (not a reference format): MLX's affine dequantization of one
 * 64-element group, w = scale * q + bias (mlx.core.dequantize, bits 4,
 * group_size 64), element 8j + i at bits 4i of little-endian code word j. */
static void dec_g64(const uint8_t* b, double w[64]) {
    double scale = hf(b), bias = hf(b + 2);
    for (int j = 0; j < 8; j++) {
        uint32_t word = rd32(b + 4 + 4 * j);
        for (int i = 0; i < 8; i++) w[8 * j + i] = (double)((word >> (4 * i)) & 15u) * scale + bias;
    }
}

static void decode_block(int f, const uint8_t* b, double* w) {
    switch (f) {
        case F_Q4_0: dec_q4_0(b, w); break;
        case F_MLX: dec_mlx(b, w); break;
        case F_Q4_K: dec_q4_k(b, w); break;
        case F_TERN: dec_tern(b, w); break;
        case F_VAR: dec_var(b, w); break;
        case F_EXL3: dec_exl3(b, w); break;
        case F_Q8_0: dec_q8_0(b, w); break;
        case F_PRISM: dec_prism(b, w); break;
        case F_G64: dec_g64(b, w); break;
    }
}

/* Dequantize a [N, K] weight matrix to fp16 bits with ONE RNE rounding of the
 * exact double value the CPU gold uses (the bit-exact dequant contract). */
EXPORT int orc_dequantize(int f, const uint8_t* W, uint16_t* out, uint32_t K, uint32_t N) {
    if (f < 0 || f > F_LAST) return -3;
    uint32_t bs = kBlockElems[f], bb = kBlockBytes[f];
    if (K % bs) return -4;
    uint32_t nb = K / bs;
    double w[256];
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t b = 0; b < nb; b++) {
            decode_block(f, W + ((size_t)n * nb + b) * bb, w);
            for (uint32_t j = 0; j < bs; j++) out[(size_t)n * K + b * bs + j] = orc_f64_to_f16(w[j]);
        }
    return 0;
}

/* Same, as the exact doubles (no rounding). */
EXPORT int orc_dequantize_f64(int f, const uint8_t* W, double* out, uint32_t K, uint32_t N) {
    if (f < 0 || f > F_LAST) return -3;
    uint32_t bs = kBlockElems[f], bb = kBlockBytes[f];
    if (K % bs) return -4;
    uint32_t nb = K / bs;
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t b = 0; b < nb; b++)
            decode_block(f, W + ((size_t)n * nb + b) * bb, out + (size_t)n * K + (size_t)b * bs);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Parallel-for over rows (replaces dispatch_apply over m)                   */
/* ------------------------------------------------------------------------ */

typedef void (*row_fn)(void* ctx, size_t row);
typedef struct { row_fn fn; void* ctx; size_t n; size_t next; pthread_mutex_t mu; } pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        size_t r = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (r >= p->n) break;
        p->fn(p->ctx, r);
    }
    return NULL;
}

static void parallel_rows(row_fn fn, void* ctx, size_t n, int nthreads) {
    if (nthreads <= 1 || n <= 1) {
        for (size_t r = 0; r < n; r++) fn(ctx, r);
        return;
    }
    if (nthreads > 256) nthreads = 256;
    pool_t p = {fn, ctx, n, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t th[256];
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, pool_worker, &p);
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* Projections: cpu_gold_reference_<fmt> (cpu_gold_reference.h:15-430)        */
/* ------------------------------------------------------------------------ */

typedef struct {
    int f;
    const uint16_t* A; const uint8_t* B; uint16_t* C; const uint16_t* R;
    uint32_t M, N, K, H, D; int direct_head;
    double* acc_out;   /* optional: raw double sums [M,N] */
} gemm_ctx;

/* Visit order of (weight index, activation index) pairs inside one block, as
 * the reference's gold loops do: interleaved (i, i+16) for the nibble formats
 * (cpu_gold_reference.h:35-41, 76-84, 135-143), sequential for ternary, EXL3,
 * PRISM, and the permuted sequential order for VAR_RATE (:312-320). */
static double block_dot(int f, const double* w, const double* a) {
    double acc = 0.0;
    switch (f) {
        case F_Q4_0: case F_MLX:
            for (int i = 0; i < 16; i++) { acc += a[i] * w[i]; acc += a[i + 16] * w[i + 16]; }
            break;
        case F_Q4_K:
            for (int s = 0; s < 8; s++)
                for (int i = 0; i < 16; i++) {
                    acc += a[s * 32 + i] * w[s * 32 + i];
                    acc += a[s * 32 + i + 16] * w[s * 32 + i + 16];
                }
            break;
        default: {
            int bs = (int)kBlockElems[f];
            for (int j = 0; j < bs; j++) acc += a[j] * w[j];
        }
    }
    return acc;
}

static void gemm_row(void* vctx, size_t m) {
    gemm_ctx* c = (gemm_ctx*)vctx;
    uint32_t bs = kBlockElems[c->f], bb = kBlockBytes[c->f], nb = c->K / bs;
    double* a = (double*)row_alloc(sizeof(double) * c->K);
    if (!a) return;
    for (uint32_t k = 0; k < c->K; k++) a[k] = orc_f16_to_f64(c->A[(size_t)m * c->K + k]);
    double w[256];
    for (uint32_t n = 0; n < c->N; n++) {
        const uint8_t* col = c->B + (size_t)n * nb * bb;
        double acc = 0.0;
        for (uint32_t b = 0; b < nb; b++) {
            decode_block(c->f, col + (size_t)b * bb, w);
            acc += block_dot(c->f, w, a + (size_t)b * bs);
        }
        if (c->acc_out) c->acc_out[(size_t)m * c->N + n] = acc;
        if (c->R) acc += orc_f16_to_f64(c->R[(size_t)m * c->N + n]);
        if (c->direct_head && c->H > 0 && c->D > 0) {
            uint32_t h = n / c->D, di = n % c->D;
            c->C[((size_t)h * c->M + m) * c->D + di] = orc_f64_to_f16(acc);
        } else {
            c->C[(size_t)m * c->N + n] = orc_f64_to_f16(acc);
        }
    }
    free(a);
}

/* C = fp16(A . W^T [+ R]) with double accumulation.  R (optional, [M,N] fp16)
 * is the residual the layer adds before its single rounding
 * (unified_prefill_engine.mm:183-186, 203-205). */
EXPORT int orc_gemm(int f, const uint16_t* A, const uint8_t* B, uint16_t* C, const uint16_t* R,
                    uint32_t M, uint32_t N, uint32_t K, int direct_head, uint32_t H, uint32_t D,
                    int nthreads) {
    if (f < 0 || f > F_LAST) return -3;
    if (K % kBlockElems[f]) return -4;
    gemm_ctx c = {f, A, B, C, R, M, N, K, H, D, direct_head, NULL};
    parallel_rows(gemm_row, &c, M, nthreads);
    return take_alloc_status();
}

/* ------------------------------------------------------------------------ */
/* brick3 fused SwiGLU gold (brick3_swiglu_bench.mm:49-99)                    */
/* ------------------------------------------------------------------------ */

typedef struct {
    int f; const uint16_t* A; const uint8_t* Bg; const uint8_t* Bu; uint16_t* O;
    uint32_t M, N, K;
} swiglu_ctx;

static void swiglu_row(void* vctx, size_t m) {
    swiglu_ctx* c = (swiglu_ctx*)vctx;
    uint32_t bs = kBlockElems[c->f], bb = kBlockBytes[c->f], nb = c->K / bs;
    double* a = (double*)row_alloc(sizeof(double) * c->K);
    if (!a) return;
    for (uint32_t k = 0; k < c->K; k++) a[k] = orc_f16_to_f64(c->A[(size_t)m * c->K + k]);
    double wg[256], wu[256];
    for (uint32_t n = 0; n < c->N; n++) {
        double ag = 0.0, au = 0.0;
        for (uint32_t b = 0; b < nb; b++) {
            decode_block(c->f, c->Bg + ((size_t)n * nb + b) * bb, wg);
            decode_block(c->f, c->Bu + ((size_t)n * nb + b) * bb, wu);
            ag += block_dot(c->f, wg, a + (size_t)b * bs);
            au += block_dot(c->f, wu, a + (size_t)b * bs);
        }
        double silu = ag / (1.0 + exp(-ag));
        c->O[(size_t)m * c->N + n] = orc_f64_to_f16(silu * au);
    }
    free(a);
}

EXPORT int orc_swiglu(int f, const uint16_t* A, const uint8_t* Bg, const uint8_t* Bu, uint16_t* O,
                      uint32_t M, uint32_t N, uint32_t K, int nthreads) {
    if (f < 0 || f > F_LAST) return -3;
    if (K % kBlockElems[f]) return -4;
    swiglu_ctx c = {f, A, Bg, Bu, O, M, N, K};
    parallel_rows(swiglu_row, &c, M, nthreads);
    return take_alloc_status();
}

/* ------------------------------------------------------------------------ */
/* Q8_0 KV quantization (brick4_attn_bench.mm:37-65; unified_kernels.metal:118-145) */
/* ------------------------------------------------------------------------ */

/* float arithmetic as in the reference: amax in float, d = amax/127 (float),
 * stored as half(d); codes use the UNROUNDED float d: q = round(x * (1/d)),
 * round half away from zero, clamped to [-128,127]. */
EXPORT void orc_quantize_q8_0(const uint16_t* src, uint8_t* dst, size_t num_blocks) {
    for (size_t b = 0; b < num_blocks; b++) {
        const uint16_t* s = src + b * 32;
        uint8_t* o = dst + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float v = fabsf(f16_to_f32(s[i]));
            if (v > amax) amax = v;
        }
        volatile float d = amax / 127.0f;
        uint16_t dh = f32_to_f16(d);
        o[0] = dh & 0xff; o[1] = dh >> 8;
        volatile float id = (d > 0.0f) ? (1.0f / d) : 0.0f;
        for (int i = 0; i < 32; i++) {
            volatile float prod = f16_to_f32(s[i]) * id;
            int q = (int)roundf(prod);
            if (q < -128) q = -128;
            if (q > 127) q = 127;
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* half(q * float(d)) per element (brick4_attn_bench.mm:57-65). */
EXPORT void orc_dequantize_q8_0(const uint8_t* src, uint16_t* dst, size_t num_blocks) {
    for (size_t b = 0; b < num_blocks; b++) {
        const uint8_t* s = src + b * 34;
        float d = f16_to_f32(rd16(s));
        for (int i = 0; i < 32; i++) {
            volatile float p = (float)(int8_t)s[2 + i] * d;
            dst[b * 32 + i] = f32_to_f16(p);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Causal attention gold (brick4_attn_bench.mm:70-119)                        */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint16_t* Q; const uint16_t* K; const uint16_t* V; uint16_t* O;
    uint32_t H, M, D; double scale; int o_token_major; uint32_t Hkv;
} attn_ctx;

static void attn_head_row(void* vctx, size_t idx) {
    attn_ctx* c = (attn_ctx*)vctx;
    size_t h = idx / c->M, i = idx % c->M;
    size_t MD = (size_t)c->M * c->D;
    size_t hk = h / (c->H / c->Hkv);  /* grouped-query: H / Hkv query heads per KV head */
    const uint16_t* q = c->Q + h * MD + i * c->D;
    double* s = (double*)row_alloc(sizeof(double) * (i + 1));
    if (!s) return;
    double mx = -1e30;
    for (size_t j = 0; j <= i; j++) {
        const uint16_t* k = c->K + hk * MD + j * c->D;
        double dot = 0.0;
        for (uint32_t d = 0; d < c->D; d++) dot += orc_f16_to_f64(q[d]) * orc_f16_to_f64(k[d]);
        s[j] = dot * c->scale;
        if (s[j] > mx) mx = s[j];
    }
    double sum = 0.0;
    for (size_t j = 0; j <= i; j++) { s[j] = exp(s[j] - mx); sum += s[j]; }
    double inv = (sum > 0.0) ? 1.0 / sum : 0.0;
    for (uint32_t d = 0; d < c->D; d++) {
        double acc = 0.0;
        for (size_t j = 0; j <= i; j++) acc += (s[j] * inv) * orc_f16_to_f64(c->V[hk * MD + j * c->D + d]);
        size_t o = c->o_token_major ? (i * (size_t)c->H + h) * c->D + d : h * MD + i * c->D + d;
        c->O[o] = orc_f64_to_f16(acc);
    }
    free(s);
}

/* Q, K, V fp16 [H, M, D]; O fp16 [H, M, D] (o_token_major = 0) or [M, H*D]
 * (o_token_major = 1, the layout the layer's O-projection consumes,
 * unified_prefill_engine.mm:171).  `scale` is the float the reference passes
 * (1/sqrt(D)), widened to double. */
EXPORT void orc_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O,
                          uint32_t H, uint32_t M, uint32_t D, float scale, int o_token_major,
                          int nthreads) {
    attn_ctx c = {Q, K, V, O, H, M, D, (double)scale, o_token_major, H};
    parallel_rows(attn_head_row, &c, (size_t)H * M, nthreads);
    if (take_alloc_status()) {
        fprintf(stderr, "oracle: out of memory in orc_attention\n");
        abort();
    }
}

/* Grouped-query attention (src/engine/model.py:234-236 passes Hkv < H heads of
 * K/V to mx.fast.scaled_dot_product_attention): query head h reads KV head
 * h / (H / Hkv).  K, V [Hkv, M, D]. */
EXPORT int orc_attention_gqa(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O,
                             uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D, float scale,
                             int o_token_major, int nthreads) {
    if (!Hkv || H % Hkv) return -4;
    attn_ctx c = {Q, K, V, O, H, M, D, (double)scale, o_token_major, Hkv};
    parallel_rows(attn_head_row, &c, (size_t)H * M, nthreads);
    return take_alloc_status();
}

/* Row-sampled causal attention: the outputs of query positions pos[0..nr)
 * only, each computed exactly as attn_head_row computes that row (the output
 * of query i depends on keys/values 0..i alone, brick4_attn_bench.mm:70-119).
 * Qr [H, nr, D] holds the sampled queries; K, V [Hkv, M, D]; Or [H, nr, D] or
 * token-major [nr, H*D].  Used to check full-size shapes on a row sample. */
typedef struct {
    const uint16_t* Q; const uint16_t* K; const uint16_t* V; uint16_t* O;
    const uint32_t* pos; uint32_t nr, H, Hkv, M, D; double scale; int o_token_major;
} attn_rows_ctx;

static void attn_rows_row(void* vctx, size_t idx) {
    attn_rows_ctx* c = (attn_rows_ctx*)vctx;
    size_t h = idx / c->nr, r = idx % c->nr, i = c->pos[r];
    size_t MD = (size_t)c->M * c->D;
    size_t hk = h / (c->H / c->Hkv);
    const uint16_t* q = c->Q + (h * c->nr + r) * c->D;
    double* s = (double*)row_alloc(sizeof(double) * (i + 1));
    if (!s) return;
    double mx = -1e30;
    for (size_t j = 0; j <= i; j++) {
        const uint16_t* k = c->K + hk * MD + j * c->D;
        double dot = 0.0;
        for (uint32_t d = 0; d < c->D; d++) dot += orc_f16_to_f64(q[d]) * orc_f16_to_f64(k[d]);
        s[j] = dot * c->scale;
        if (s[j] > mx) mx = s[j];
    }
    double sum = 0.0;
    for (size_t j = 0; j <= i; j++) { s[j] = exp(s[j] - mx); sum += s[j]; }
    double inv = (sum > 0.0) ? 1.0 / sum : 0.0;
    for (uint32_t d = 0; d < c->D; d++) {
        double acc = 0.0;
        for (size_t j = 0; j <= i; j++) acc += (s[j] * inv) * orc_f16_to_f64(c->V[hk * MD + j * c->D + d]);
        size_t o = c->o_token_major ? (r * (size_t)c->H + h) * c->D + d : (h * c->nr + r) * c->D + d;
        c->O[o] = orc_f64_to_f16(acc);
    }
    free(s);
}

EXPORT int orc_attention_rows(const uint16_t* Qr, const uint16_t* K, const uint16_t* V, uint16_t* Or,
                              const uint32_t* pos, uint32_t nr, uint32_t H, uint32_t Hkv, uint32_t M,
                              uint32_t D, float scale, int o_token_major, int nthreads) {
    if (!Hkv || H % Hkv) return -4;
    for (uint32_t r = 0; r < nr; r++)
        if (pos[r] >= M) return -4;
    attn_rows_ctx c = {Qr, K, V, Or, pos, nr, H, Hkv, M, D, (double)scale, o_token_major};
    parallel_rows(attn_rows_row, &c, (size_t)H * nr, nthreads);
    return take_alloc_status();
}

/* Attention over a Q8_0 KV cache: the reference checks its Q8_0 kernel
 * against the double gold run on the DEQUANTIZED K/V
 * (brick4_attn_bench.mm:241-255).  Kq/Vq are Q8_0 blocks over [H, M, D]. */
EXPORT void orc_attention_q8_0(const uint16_t* Q, const uint8_t* Kq, const uint8_t* Vq, uint16_t* O,
                               uint32_t H, uint32_t M, uint32_t D, float scale, int o_token_major,
                               int nthreads) {
    size_t n = (size_t)H * M * D;
    uint16_t* Kd = (uint16_t*)must_alloc(n * 2);
    uint16_t* Vd = (uint16_t*)must_alloc(n * 2);
    orc_dequantize_q8_0(Kq, Kd, n / 32);
    orc_dequantize_q8_0(Vq, Vd, n / 32);
    orc_attention(Q, Kd, Vd, O, H, M, D, scale, o_token_major, nthreads);
    free(Kd);
    free(Vd);
}

/* Same with Hkv KV heads (Kq/Vq blocks over [Hkv, M, D]). */
EXPORT int orc_attention_q8_0_gqa(const uint16_t* Q, const uint8_t* Kq, const uint8_t* Vq, uint16_t* O,
                                  uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D, float scale,
                                  int o_token_major, int nthreads) {
    size_t n = (size_t)Hkv * M * D;
    uint16_t* Kd = (uint16_t*)must_alloc(n * 2);
    uint16_t* Vd = (uint16_t*)must_alloc(n * 2);
    orc_dequantize_q8_0(Kq, Kd, n / 32);
    orc_dequantize_q8_0(Vq, Vd, n / 32);
    int rc = orc_attention_gqa(Q, Kd, Vd, O, H, Hkv, M, D, scale, o_token_major, nthreads);
    free(Kd);
    free(Vd);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* RMSNorm and RoPE of the MLX block (src/engine/model.py:17-48, :112-116,   */
/* :215-226), restated in double with the fp16 rounding points of the model  */
/* ------------------------------------------------------------------------ */

/* RMSNorm over rows of X [M, D] (model.py:39-48):
 *   normed = fp16(x / sqrt(mean(x^2) + eps))
 *   y      = fp16(normed * w)               norm_type 1 ("rmsnorm")
 *   y      = fp16(normed * fp16(1 + w))     norm_type 2 ("gemma_add_one")
 * The mean and root are taken in double (the model: float32). */
EXPORT int orc_rmsnorm(const uint16_t* X, const uint16_t* w, uint16_t* Y, uint32_t M, uint32_t D,
                       float eps, int norm_type) {
    if (norm_type != 1 && norm_type != 2) return -3;
    for (uint32_t m = 0; m < M; m++) {
        const uint16_t* x = X + (size_t)m * D;
        double ss = 0.0;
        for (uint32_t d = 0; d < D; d++) {
            double v = orc_f16_to_f64(x[d]);
            ss += v * v;
        }
        double r = 1.0 / sqrt(ss / (double)D + (double)eps);
        for (uint32_t d = 0; d < D; d++) {
            double nv = orc_f16_to_f64(orc_f64_to_f16(orc_f16_to_f64(x[d]) * r));
            double wv = orc_f16_to_f64(w[d]);
            if (norm_type == 2) wv = orc_f16_to_f64(orc_f64_to_f16(1.0 + wv));
            Y[(size_t)m * D + d] = orc_f64_to_f16(nv * wv);
        }
    }
    return 0;
}

/* Rotary position embedding in place on T [H, M, D] (nn.RoPE(dims = D,
 * traditional, base = theta) at model.py:112-116, applied with the cache
 * offset at :218-219).  Row m has position offset + m; pair i (0 <= i < D/2)
 * rotates by angle pos * theta^(-2i/D): elements (i, i + D/2), or (2i, 2i+1)
 * when traditional:  a' = a cos - b sin,  b' = a sin + b cos, each rounded to
 * fp16 once. */
EXPORT int orc_rope(uint16_t* T, uint32_t H, uint32_t M, uint32_t D, float theta, uint32_t offset,
                    int traditional) {
    if (D % 2) return -4;
    uint32_t half = D / 2;
    for (size_t r = 0; r < (size_t)H * M; r++) {
        uint16_t* t = T + r * D;
        double pos = (double)(offset + (uint32_t)(r % M));
        for (uint32_t i = 0; i < half; i++) {
            double ang = pos * pow((double)theta, -2.0 * (double)i / (double)D);
            double c = cos(ang), sn = sin(ang);
            uint32_t ia = traditional ? 2 * i : i, ib = traditional ? 2 * i + 1 : i + half;
            double a = orc_f16_to_f64(t[ia]), b = orc_f16_to_f64(t[ib]);
            t[ia] = orc_f64_to_f16(a * c - b * sn);
            t[ib] = orc_f64_to_f16(a * sn + b * c);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* One prefill layer (unified_prefill_engine.mm:72-223, restated in double)   */
/* ------------------------------------------------------------------------ */

/*
 * X_out = L(X) for one Llama-style prefill layer with no norm and no RoPE, as
 * the reference's layer reference and coordinator compose it
 * (unified_prefill_engine.mm:72-223; models/transformer_layer.mm:75-218):
 *   Q,K,V = fp16(X . Wq/k/v^T) written head-major [H, M, D]
 *   Kq,Vq = Q8_0(K), Q8_0(V)                  (unified_prefill_engine.mm:554-572)
 *   O     = fp16(causal_attn(Q, deq Kq, deq Vq)) token-major [M, H*D]
 *   Xmid  = fp16(X + O . Wo^T)                 (one rounding, :183-186)
 *   S     = fp16(silu(Xmid . Wg^T) * (Xmid . Wu^T))  (double epilogue)
 *   Xout  = fp16(Xmid + S . Wd^T)              (one rounding, :203-205)
 * The reference's layer reference accumulates in float; this restatement
 * accumulates in double with the rounding points of the GPU pipeline.
 * Optional outputs (may be NULL): Qh, Kh, Vh [H,M,D]; Oattn [M,HD]; Xmid
 * [M,dm]; S [M,Nm].
 */
EXPORT int orc_layer(int f, const uint16_t* X, const uint8_t* Wq, const uint8_t* Wk,
                     const uint8_t* Wv, const uint8_t* Wo, const uint8_t* Wg, const uint8_t* Wu,
                     const uint8_t* Wd, uint16_t* Xout, uint32_t M, uint32_t dm, uint32_t H,
                     uint32_t D, uint32_t Nm, float scale, uint16_t* Qh, uint16_t* Kh,
                     uint16_t* Vh, uint16_t* Oattn, uint16_t* Xmid, uint16_t* S, int nthreads) {
    uint32_t HD = H * D;
    size_t nq = (size_t)M * HD;
    uint16_t* q = Qh ? Qh : (uint16_t*)must_alloc(nq * 2);
    uint16_t* k = Kh ? Kh : (uint16_t*)must_alloc(nq * 2);
    uint16_t* v = Vh ? Vh : (uint16_t*)must_alloc(nq * 2);
    uint16_t* o = Oattn ? Oattn : (uint16_t*)must_alloc(nq * 2);
    uint16_t* xm = Xmid ? Xmid : (uint16_t*)must_alloc((size_t)M * dm * 2);
    uint16_t* s = S ? S : (uint16_t*)must_alloc((size_t)M * Nm * 2);
    uint8_t* kq = (uint8_t*)must_alloc(nq / 32 * 34);
    uint8_t* vq = (uint8_t*)must_alloc(nq / 32 * 34);
    int rc = 0;
    rc |= orc_gemm(f, X, Wq, q, NULL, M, HD, dm, 1, H, D, nthreads);
    rc |= orc_gemm(f, X, Wk, k, NULL, M, HD, dm, 1, H, D, nthreads);
    rc |= orc_gemm(f, X, Wv, v, NULL, M, HD, dm, 1, H, D, nthreads);
    orc_quantize_q8_0(k, kq, nq / 32);
    orc_quantize_q8_0(v, vq, nq / 32);
    orc_attention_q8_0(q, kq, vq, o, H, M, D, scale, 1, nthreads);
    rc |= orc_gemm(f, o, Wo, xm, X, M, dm, HD, 0, 0, 0, nthreads);
    rc |= orc_swiglu(f, xm, Wg, Wu, s, M, Nm, dm, nthreads);
    rc |= orc_gemm(f, s, Wd, Xout, xm, M, dm, Nm, 0, 0, 0, nthreads);
    if (!Qh) free(q);
    if (!Kh) free(k);
    if (!Vh) free(v);
    if (!Oattn) free(o);
    if (!Xmid) free(xm);
    if (!S) free(s);
    free(kq);
    free(vq);
    return rc;
}

/*
 * The MLX block with the router's projections (src/engine/model.py:181-265):
 *   Xn    = RMSNorm(X, w_attn)                 (skipped when w_attn is NULL)
 *   Q     = fp16(Xn . Wq^T) [Hq, M, D];  K, V = fp16(Xn . Wk/v^T) [Hkv, M, D]
 *   Q, K  = RoPE(Q), RoPE(K) at positions offset + m   (skipped if !rope)
 *   O     = fp16(causal_attn_gqa(Q, deq Q8_0(K), deq Q8_0(V))) token-major
 *   Xmid  = fp16(X + O . Wo^T)
 *   Xn2   = RMSNorm(Xmid, w_ffn)               (skipped when w_ffn is NULL)
 *   S     = fp16(silu(Xn2 . Wg^T) * (Xn2 . Wu^T))
 *   Xout  = fp16(Xmid + S . Wd^T)
 * The KV cache is Q8_0 as in the router's layer (unified_prefill_engine.mm:
 * 554-572); rounding points are those of the GPU pipeline.
 */
EXPORT int orc_layer_ex(int f, const uint16_t* X, const uint16_t* w_attn, const uint8_t* Wq,
                        const uint8_t* Wk, const uint8_t* Wv, const uint8_t* Wo, const uint16_t* w_ffn,
                        const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, uint16_t* Xout,
                        uint32_t M, uint32_t dm, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t Nm,
                        float scale, int norm_type, float eps, int rope, float theta, uint32_t offset,
                        int traditional, int nthreads) {
    if (!Hkv || Hq % Hkv) return -4;
    uint32_t HQ = Hq * D, HK = Hkv * D;
    size_t nq = (size_t)M * HQ, nk = (size_t)M * HK;
    uint16_t* xn = (uint16_t*)must_alloc((size_t)M * dm * 2);
    uint16_t* q = (uint16_t*)must_alloc(nq * 2);
    uint16_t* k = (uint16_t*)must_alloc(nk * 2);
    uint16_t* v = (uint16_t*)must_alloc(nk * 2);
    uint16_t* o = (uint16_t*)must_alloc(nq * 2);
    uint16_t* xm = (uint16_t*)must_alloc((size_t)M * dm * 2);
    uint16_t* s = (uint16_t*)must_alloc((size_t)M * Nm * 2);
    uint8_t* kq = (uint8_t*)must_alloc(nk / 32 * 34);
    uint8_t* vq = (uint8_t*)must_alloc(nk / 32 * 34);
    int rc = 0;
    const uint16_t* a = X;
    if (w_attn) {
        rc |= orc_rmsnorm(X, w_attn, xn, M, dm, eps, norm_type);
        a = xn;
    }
    rc |= orc_gemm(f, a, Wq, q, NULL, M, HQ, dm, 1, Hq, D, nthreads);
    rc |= orc_gemm(f, a, Wk, k, NULL, M, HK, dm, 1, Hkv, D, nthreads);
    rc |= orc_gemm(f, a, Wv, v, NULL, M, HK, dm, 1, Hkv, D, nthreads);
    if (rope) {
        rc |= orc_rope(q, Hq, M, D, theta, offset, traditional);
        rc |= orc_rope(k, Hkv, M, D, theta, offset, traditional);
    }
    orc_quantize_q8_0(k, kq, nk / 32);
    orc_quantize_q8_0(v, vq, nk / 32);
    rc |= orc_attention_q8_0_gqa(q, kq, vq, o, Hq, Hkv, M, D, scale, 1, nthreads);
    rc |= orc_gemm(f, o, Wo, xm, X, M, dm, HQ, 0, 0, 0, nthreads);
    a = xm;
    if (w_ffn) {
        rc |= orc_rmsnorm(xm, w_ffn, xn, M, dm, eps, norm_type);
        a = xn;
    }
    rc |= orc_swiglu(f, a, Wg, Wu, s, M, Nm, dm, nthreads);
    rc |= orc_gemm(f, s, Wd, Xout, xm, M, dm, Nm, 0, 0, 0, nthreads);
    free(xn); free(q); free(k); free(v); free(o); free(xm); free(s); free(kq); free(vq);
    return rc;
}

/*
 * orc_layer_ex on a row sample: Xout rows pos[0..nr) only.  Row m of the
 * layer depends on row m of X and on the K / V of rows 0..m, so K and V are
 * projected (and Q8_0-quantized) for every row while Q, attention, the
 * O-projection, the norms and the MLP run on the sampled rows alone -- the
 * same arithmetic, row by row, as orc_layer_ex.  Xout [nr, dm].
 */
EXPORT int orc_layer_ex_rows(int f, const uint16_t* X, const uint16_t* w_attn, const uint8_t* Wq,
                             const uint8_t* Wk, const uint8_t* Wv, const uint8_t* Wo, const uint16_t* w_ffn,
                             const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd, uint16_t* Xout,
                             const uint32_t* pos, uint32_t nr, uint32_t M, uint32_t dm, uint32_t Hq,
                             uint32_t Hkv, uint32_t D, uint32_t Nm, float scale, int norm_type, float eps,
                             int rope, float theta, uint32_t offset, int traditional, int nthreads) {
    if (!Hkv || Hq % Hkv) return -4;
    for (uint32_t r = 0; r < nr; r++)
        if (pos[r] >= M) return -4;
    uint32_t HQ = Hq * D, HK = Hkv * D;
    size_t nk = (size_t)M * HK;
    uint16_t* xn = (uint16_t*)must_alloc((size_t)M * dm * 2);
    uint16_t* k = (uint16_t*)must_alloc(nk * 2);
    uint16_t* v = (uint16_t*)must_alloc(nk * 2);
    uint8_t* kq = (uint8_t*)must_alloc(nk / 32 * 34);
    uint8_t* vq = (uint8_t*)must_alloc(nk / 32 * 34);
    uint16_t* xr = (uint16_t*)must_alloc((size_t)nr * dm * 2);    /* sampled (normed) rows */
    uint16_t* x0 = (uint16_t*)must_alloc((size_t)nr * dm * 2);    /* sampled input rows */
    uint16_t* q = (uint16_t*)must_alloc((size_t)nr * HQ * 2);
    uint16_t* o = (uint16_t*)must_alloc((size_t)nr * HQ * 2);
    uint16_t* xm = (uint16_t*)must_alloc((size_t)nr * dm * 2);
    uint16_t* xn2 = (uint16_t*)must_alloc((size_t)nr * dm * 2);
    uint16_t* s = (uint16_t*)must_alloc((size_t)nr * Nm * 2);
    int rc = 0;
    const uint16_t* a = X;
    if (w_attn) {
        rc |= orc_rmsnorm(X, w_attn, xn, M, dm, eps, norm_type);
        a = xn;
    }
    for (uint32_t r = 0; r < nr; r++) {
        memcpy(xr + (size_t)r * dm, a + (size_t)pos[r] * dm, (size_t)dm * 2);
        memcpy(x0 + (size_t)r * dm, X + (size_t)pos[r] * dm, (size_t)dm * 2);
    }
    rc |= orc_gemm(f, a, Wk, k, NULL, M, HK, dm, 1, Hkv, D, nthreads);
    rc |= orc_gemm(f, a, Wv, v, NULL, M, HK, dm, 1, Hkv, D, nthreads);
    rc |= orc_gemm(f, xr, Wq, q, NULL, nr, HQ, dm, 1, Hq, D, nthreads);   /* [Hq, nr, D] */
    if (rope) {
        /* the sampled query rows rotate at their own positions */
        for (uint32_t r = 0; r < nr; r++)
            for (uint32_t h = 0; h < Hq; h++)
                rc |= orc_rope(q + ((size_t)h * nr + r) * D, 1, 1, D, theta, offset + pos[r], traditional);
        rc |= orc_rope(k, Hkv, M, D, theta, offset, traditional);
    }
    orc_quantize_q8_0(k, kq, nk / 32);
    orc_quantize_q8_0(v, vq, nk / 32);
    orc_dequantize_q8_0(kq, k, nk / 32);
    orc_dequantize_q8_0(vq, v, nk / 32);
    rc |= orc_attention_rows(q, k, v, o, pos, nr, Hq, Hkv, M, D, scale, 1, nthreads);
    rc |= orc_gemm(f, o, Wo, xm, x0, nr, dm, HQ, 0, 0, 0, nthreads);
    a = xm;
    if (w_ffn) {
        rc |= orc_rmsnorm(xm, w_ffn, xn2, nr, dm, eps, norm_type);
        a = xn2;
    }
    rc |= orc_swiglu(f, a, Wg, Wu, s, nr, Nm, dm, nthreads);
    rc |= orc_gemm(f, s, Wd, Xout, xm, nr, dm, Nm, 0, 0, 0, nthreads);
    free(xn); free(k); free(v); free(kq); free(vq); free(xr); free(x0); free(q); free(o);
    free(xm); free(xn2); free(s);
    return rc;
}
