/*
 * CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE ONLY (see w4a16_oracle.h).
 *
 * Restates, in plain C, the arithmetic of the reference's int4 weight-only GEMM and
 * dequant kernels:
 *   crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs   (GPTQ GEMM)
 *   crates/triton-dsl/examples/awq_gemm_int4_typed.rs     (AWQ GEMM)
 *   crates/triton-dsl/examples/ferrum_dequant_int4.rs     (GPTQ asym dequant)
 *   crates/triton-dsl/examples/ferrum_dequant_int4_sym.rs (GPTQ sym dequant)
 * act-order (g_idx) and the fused MoE are not in the reference; they are defined here
 * by composition of the above and pinned by the invariants in tests/test_oracle*.py.
 */
#include "w4a16_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu;
    const uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFFu) {                      /* inf / nan */
        if (mant == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (mant >> 13)); /* quiet NaN */
    }
    const int e = (int)exp - 127 + 15;       /* biased f16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e >= 1) {                            /* normal range (may round up to inf) */
        uint32_t r = ((uint32_t)e << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u;
        return (uint16_t)(sign | r);
    }
    if (exp == 0) return (uint16_t)sign;     /* f32 zero / subnormal: far below f16 range */
    /* f16 subnormal: count units of 2^-24. value = m * 2^(exp-150), units = m >> (126-exp) */
    const uint32_t m = mant | 0x800000u;
    const int shift = 14 - e;                /* == 126 - exp, >= 14 here */
    if (shift >= 25) return (uint16_t)sign;  /* < half of the smallest subnormal (or = half: even 0) */
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r += 1u;
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (exp == 0x1Fu) {
        x = sign | 0x7F800000u | (mant << 13);
    } else if (exp != 0) {
        x = sign | ((exp - 15u + 127u) << 23) | (mant << 13);
    } else if (mant == 0) {
        x = sign;
    } else {                                 /* subnormal: normalise */
        int e = -1;
        do { mant <<= 1; e++; } while ((mant & 0x400u) == 0);
        mant &= 0x3FFu;
        x = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static float g_f16_lut[65536];

__attribute__((constructor)) static void orc_init_lut(void) {
    for (uint32_t i = 0; i < 65536u; ++i) g_f16_lut[i] = orc_f16_to_f32((uint16_t)i);
}

static inline float h2f(uint16_t h) { return g_f16_lut[h]; }

void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = h2f(src[i]);
}

/* ------------------------------------------------------------------ bf16 */
/* The reference kernels are generic over the element type T and name bf16
 * (w4a16_gptq_gemm_typed.rs:65-67); as_t::<bf16>(f32) is arith.truncf, round to nearest even
 * (module.rs:726-731). bfloat16 is the top half of an f32. */

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu))
        return (uint16_t)((x >> 16) | 0x40u);      /* NaN stays NaN (quiet), sign kept */
    x += 0x7FFFu + ((x >> 16) & 1u);               /* to nearest, ties to even; may reach inf */
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}

void orc_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* element type of the 16-bit operands: 0 fp16, 1 bf16 */
static inline float e2f(uint16_t v, int bf16) { return bf16 ? orc_bf16_to_f32(v) : h2f(v); }
static inline uint16_t f2e(float v, int bf16) { return bf16 ? orc_f32_to_bf16(v) : orc_f32_to_f16(v); }

/* ------------------------------------------------------------ unpacking */

int orc_awq_slot(int n) {
    /* awq_gemm_int4_typed.rs:139-151: awq_lane = (n%8)/2 + ((n%8)%2)*4 */
    const int l = n % 8;
    return l / 2 + (l % 2) * 4;
}

int orc_nibble(int32_t word, int slot) {
    /* shr_u_i32 = arith.shrui (logical), then bit_and 0xF */
    return (int)(((uint32_t)word >> (4 * slot)) & 0xFu);
}

int orc_qweight_at(int fmt, const int32_t* qweight, int K, int N, int k, int n) {
    (void)K;
    if (fmt == ORC_FMT_AWQ) {
        /* qweight [K, N/8]; lane (k, n) reads qweight[k, n/8] (awq_gemm_int4_typed.rs:189-195) */
        return orc_nibble(qweight[(size_t)k * (N / 8) + n / 8], orc_awq_slot(n));
    }
    /* qweight [K/8, N]; lane (k, n) reads qweight[k/8, n], shift (k%8)*4
     * (w4a16_gptq_gemm_typed.rs:175-180, 213-217) */
    return orc_nibble(qweight[(size_t)(k / 8) * N + n], k % 8);
}

int orc_zero_at(int fmt, const int32_t* qzeros, int N, int g, int n, int zero_offset) {
    if (fmt == ORC_FMT_GPTQ_SYM) return 8;               /* ferrum_dequant_int4_sym.rs:60 */
    const int32_t word = qzeros[(size_t)g * (N / 8) + n / 8];
    if (fmt == ORC_FMT_AWQ) return orc_nibble(word, orc_awq_slot(n)); /* awq :203-205 */
    return orc_nibble(word, n % 8) + zero_offset;        /* gptq :231-236 (+1) */
}

static inline uint16_t dequant_one(int q, int z, uint16_t s, int bf16) {
    /* to_f32(centered) * to_f32(scale) then as_t::<T> = truncf (RNE):
     * w4a16_gptq_gemm_typed.rs:256-260, awq_gemm_int4_typed.rs:224-228 */
    return f2e((float)(q - z) * e2f(s, bf16), bf16);
}

static int check_gidx(const int32_t* g_idx, int K, int N, int G) {
    if (!g_idx) return 0;
    const int ngroups = K / G;
    for (int k = 0; k < K; ++k)
        if (g_idx[k] < 0 || g_idx[k] >= ngroups) return -1;
    (void)N;
    return 0;
}

static int dequant_impl(int fmt, const int32_t* qweight, const uint16_t* scales,
                        const int32_t* qzeros, const int32_t* g_idx, int K, int N, int G,
                        int zero_offset, int bf16, uint16_t* out) {
    if (check_gidx(g_idx, K, N, G)) return -1;
#pragma omp parallel for schedule(static)
    for (int k = 0; k < K; ++k) {
        const int g = g_idx ? g_idx[k] : k / G;
        for (int n = 0; n < N; ++n) {
            const int q = orc_qweight_at(fmt, qweight, K, N, k, n);
            const int z = orc_zero_at(fmt, qzeros, N, g, n, zero_offset);
            out[(size_t)k * N + n] = dequant_one(q, z, scales[(size_t)g * N + n], bf16);
        }
    }
    return 0;
}

int orc_dequant(int fmt, const int32_t* qweight, const uint16_t* scales,
                const int32_t* qzeros, const int32_t* g_idx, int K, int N, int G,
                int zero_offset, uint16_t* out) {
    return dequant_impl(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, 0, out);
}

int orc_dequant_bf16(int fmt, const int32_t* qweight, const uint16_t* scales,
                     const int32_t* qzeros, const int32_t* g_idx, int K, int N, int G,
                     int zero_offset, uint16_t* out) {
    return dequant_impl(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, 1, out);
}

static int dequant_transposed_impl(int fmt, const int32_t* qweight, const uint16_t* scales,
                                   const int32_t* qzeros, const int32_t* g_idx, int K, int N,
                                   int G, int zero_offset, int bf16, uint16_t* out_nk) {
    if (check_gidx(g_idx, K, N, G)) return -1;
    /* ferrum_dequant_int4.rs:121-138: store(output + col*K + base_k + i) */
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        for (int k = 0; k < K; ++k) {
            const int g = g_idx ? g_idx[k] : k / G;
            const int q = orc_qweight_at(fmt, qweight, K, N, k, n);
            const int z = orc_zero_at(fmt, qzeros, N, g, n, zero_offset);
            out_nk[(size_t)n * K + k] = dequant_one(q, z, scales[(size_t)g * N + n], bf16);
        }
    }
    return 0;
}

int orc_dequant_transposed(int fmt, const int32_t* qweight, const uint16_t* scales,
                           const int32_t* qzeros, const int32_t* g_idx, int K, int N,
                           int G, int zero_offset, uint16_t* out_nk) {
    return dequant_transposed_impl(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, 0,
                                   out_nk);
}

int orc_dequant_transposed_bf16(int fmt, const int32_t* qweight, const uint16_t* scales,
                                const int32_t* qzeros, const int32_t* g_idx, int K, int N,
                                int G, int zero_offset, uint16_t* out_nk) {
    return dequant_transposed_impl(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, 1,
                                   out_nk);
}

/* ---------------------------------------------------------------- GEMM */

#define COLBLK 256

static void gemm_rows(const uint16_t* x, const uint16_t* w16, const int32_t* rows,
                      int nrows, int N, int K, int acc64, int bf16, uint16_t* out,
                      float* out_f32) {
    const int nblk = (N + COLBLK - 1) / COLBLK;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (int ri = 0; ri < nrows; ++ri) {
        for (int b = 0; b < nblk; ++b) {
            const int m = rows ? rows[ri] : ri;
            const int n0 = b * COLBLK;
            const int n1 = n0 + COLBLK < N ? n0 + COLBLK : N;
            const uint16_t* xr = x + (size_t)m * K;
            if (acc64) {
                double acc[COLBLK];
                for (int n = n0; n < n1; ++n) acc[n - n0] = 0.0;
                for (int k = 0; k < K; ++k) {
                    const double xv = (double)e2f(xr[k], bf16);
                    const uint16_t* wr = w16 + (size_t)k * N;
                    for (int n = n0; n < n1; ++n) acc[n - n0] += xv * (double)e2f(wr[n], bf16);
                }
                for (int n = n0; n < n1; ++n) {
                    const float v = (float)acc[n - n0];
                    out[(size_t)ri * N + n] = f2e(v, bf16);
                    if (out_f32) out_f32[(size_t)ri * N + n] = v;
                }
            } else {
                float acc[COLBLK];
                for (int n = n0; n < n1; ++n) acc[n - n0] = 0.0f;
                for (int k = 0; k < K; ++k) {
                    const float xv = e2f(xr[k], bf16);
                    const uint16_t* wr = w16 + (size_t)k * N;
                    for (int n = n0; n < n1; ++n) acc[n - n0] += xv * e2f(wr[n], bf16);
                }
                for (int n = n0; n < n1; ++n) {
                    out[(size_t)ri * N + n] = f2e(acc[n - n0], bf16);
                    if (out_f32) out_f32[(size_t)ri * N + n] = acc[n - n0];
                }
            }
        }
    }
}

void orc_gemm_f16(const uint16_t* x, const uint16_t* w16, int M, int N, int K,
                  int acc64, uint16_t* out, float* out_f32) {
    gemm_rows(x, w16, NULL, M, N, K, acc64, 0, out, out_f32);
}

int orc_w4a16_gemm(int fmt, const uint16_t* x, const int32_t* qweight,
                   const uint16_t* scales, const int32_t* qzeros, const int32_t* g_idx,
                   int M, int N, int K, int G, int zero_offset, int acc64,
                   uint16_t* out, float* out_f32) {
    uint16_t* w16 = (uint16_t*)malloc((size_t)K * N * sizeof(uint16_t));
    if (!w16) return -2;
    int rc = orc_dequant(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, w16);
    if (rc == 0) orc_gemm_f16(x, w16, M, N, K, acc64, out, out_f32);
    free(w16);
    return rc;
}

int orc_w4a16_gemm_bf16(int fmt, const uint16_t* x, const int32_t* qweight,
                        const uint16_t* scales, const int32_t* qzeros, const int32_t* g_idx,
                        int M, int N, int K, int G, int zero_offset, int acc64,
                        uint16_t* out, float* out_f32) {
    uint16_t* w16 = (uint16_t*)malloc((size_t)K * N * sizeof(uint16_t));
    if (!w16) return -2;
    int rc = dequant_impl(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, 1, w16);
    if (rc == 0) gemm_rows(x, w16, NULL, M, N, K, acc64, 1, out, out_f32);
    free(w16);
    return rc;
}

int orc_w4a16_gemm_rows(int fmt, const uint16_t* x, const int32_t* qweight,
                        const uint16_t* scales, const int32_t* qzeros,
                        const int32_t* g_idx, int M, int N, int K, int G,
                        int zero_offset, const int32_t* rows, int nrows, uint16_t* out) {
    for (int i = 0; i < nrows; ++i)
        if (rows[i] < 0 || rows[i] >= M) return -1;
    uint16_t* w16 = (uint16_t*)malloc((size_t)K * N * sizeof(uint16_t));
    if (!w16) return -2;
    int rc = orc_dequant(fmt, qweight, scales, qzeros, g_idx, K, N, G, zero_offset, w16);
    if (rc == 0) gemm_rows(x, w16, rows, nrows, N, K, 1, 0, out, NULL);
    free(w16);
    return rc;
}

/* ----------------------------------------------------------------- MoE */

void orc_moe_route(const float* logits, int T, int E, int topk, int32_t* ids, float* weights) {
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t)t * E;
        float mx = l[0];
        for (int e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
        double p[256];
        double sum = 0.0;
        for (int e = 0; e < E; ++e) { p[e] = exp((double)(l[e] - mx)); sum += p[e]; }
        for (int e = 0; e < E; ++e) p[e] /= sum;
        int used[256] = {0};
        double wsum = 0.0;
        for (int j = 0; j < topk; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (used[e]) continue;
                if (best < 0 || p[e] > p[best]) best = e;   /* strict >: ties keep lower index */
            }
            used[best] = 1;
            ids[(size_t)t * topk + j] = best;
            weights[(size_t)t * topk + j] = (float)p[best];
            wsum += p[best];
        }
        for (int j = 0; j < topk; ++j)
            weights[(size_t)t * topk + j] = (float)((double)weights[(size_t)t * topk + j] / wsum);
    }
}

int orc_moe_align(const int32_t* ids, int T, int topk, int E, int block_m,
                  int32_t* sorted_ids, int32_t* expert_ids) {
    const int P = T * topk;
    int* cnt = (int*)calloc((size_t)E, sizeof(int));
    for (int p = 0; p < P; ++p) cnt[ids[p]]++;
    int total = 0;
    int* start = (int*)malloc((size_t)E * sizeof(int));
    for (int e = 0; e < E; ++e) {
        start[e] = total;
        const int padded = (cnt[e] + block_m - 1) / block_m * block_m;
        for (int b = 0; b < padded / block_m; ++b) expert_ids[(total / block_m) + b] = e;
        for (int i = 0; i < padded; ++i) sorted_ids[total + i] = P;   /* sentinel */
        total += padded;
    }
    int* fill = (int*)calloc((size_t)E, sizeof(int));
    for (int p = 0; p < P; ++p) {
        const int e = ids[p];
        sorted_ids[start[e] + fill[e]++] = p;
    }
    free(cnt); free(start); free(fill);
    return total;
}

/* crates/triton-kernels/src/elementwise.rs:214-250: denom = exp(-g) + 1, silu = g / denom,
 * out = silu * u, every step in f32. */
float orc_silu_mul_f32(float g, float u) {
    const float denom = expf(-g) + 1.0f;
    const float s = g / denom;
    return s * u;
}

void orc_silu_mul_f32_rows(const float* gate_up, float* out, int inter, int64_t total) {
    for (int64_t i = 0; i < total; ++i) {
        const int64_t b = i / inter, c = i % inter;
        out[i] = orc_silu_mul_f32(gate_up[b * 2 * inter + c], gate_up[b * 2 * inter + inter + c]);
    }
}

uint16_t orc_silu_mul_f16(uint16_t g, uint16_t u) {
    const float gf = h2f(g);
    const float s = gf / (1.0f + expf(-gf));
    return orc_f32_to_f16(s * h2f(u));
}

void orc_moe_forward(const uint16_t* x, int T, int K, int I, int E, int topk,
                     const int32_t* ids, const float* weights,
                     const uint16_t* const* w13, const uint16_t* const* w2, uint16_t* y) {
    (void)E;
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < T; ++t) {
        float* h = (float*)malloc((size_t)2 * I * sizeof(float));
        uint16_t* a = (uint16_t*)malloc((size_t)I * sizeof(uint16_t));
        float* ye = (float*)malloc((size_t)K * sizeof(float));
        double* yacc = (double*)calloc((size_t)K, sizeof(double));
        const uint16_t* xr = x + (size_t)t * K;
        for (int j = 0; j < topk; ++j) {
            const int e = ids[(size_t)t * topk + j];
            const float w = weights[(size_t)t * topk + j];
            const uint16_t* W13 = w13[e];
            for (int n = 0; n < 2 * I; ++n) h[n] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float xv = h2f(xr[k]);
                const uint16_t* wr = W13 + (size_t)k * 2 * I;
                for (int n = 0; n < 2 * I; ++n) h[n] += xv * h2f(wr[n]);
            }
            for (int i = 0; i < I; ++i)
                a[i] = orc_silu_mul_f16(orc_f32_to_f16(h[i]), orc_f32_to_f16(h[I + i]));
            const uint16_t* W2 = w2[e];
            for (int n = 0; n < K; ++n) ye[n] = 0.0f;
            for (int i = 0; i < I; ++i) {
                const float av = h2f(a[i]);
                const uint16_t* wr = W2 + (size_t)i * K;
                for (int n = 0; n < K; ++n) ye[n] += av * h2f(wr[n]);
            }
            for (int n = 0; n < K; ++n)
                yacc[n] += (double)w * (double)h2f(orc_f32_to_f16(ye[n]));
        }
        for (int n = 0; n < K; ++n) y[(size_t)t * K + n] = orc_f32_to_f16((float)yacc[n]);
        free(h); free(a); free(ye); free(yacc);
    }
}

/* ------------------------------------------------------------- threads */

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
