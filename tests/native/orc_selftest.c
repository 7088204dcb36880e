/* The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: every entry point on
 * small inputs, including edge shapes (one row, one group, K = 8, column tails), checked for
 * memory errors and undefined behaviour, plus cross-checks that need no second
 * implementation: fp16 round trips, the known nibble orders, dequant = (q - z) * s on exact
 * values, the dense GEMM of a one-hot row equals that row of W16, GPTQ with qzeros 0x77777777
 * (+1) equals GPTQ_SYM, route weights summing to 1, align listing every pair once.
 * Exit status 0 = all passed. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "w4a16_oracle.h"

static int failures = 0;
#define CHECK(c) do { if (!(c)) { fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); ++failures; } } while (0)

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return (uint32_t)(rs >> 16); }

static void fill_words(int32_t* w, size_t n) { for (size_t i = 0; i < n; ++i) w[i] = (int32_t)rnd(); }
static void fill_scales(uint16_t* s, size_t n) {
    for (size_t i = 0; i < n; ++i) s[i] = orc_f32_to_f16(0.002f + 0.018f * (float)(rnd() % 1000) / 1000.0f);
}
static void fill_x(uint16_t* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_f32_to_f16(((float)(rnd() % 2001) - 1000.0f) / 500.0f);
}

static void test_f16(void) {
    for (uint32_t h = 0; h < 65536; ++h) {
        const float f = orc_f16_to_f32((uint16_t)h);
        if (isnan(f)) continue;
        CHECK(orc_f32_to_f16(f) == h);
    }
    CHECK(orc_f32_to_f16(65520.0f) == 0x7C00);      /* rounds to infinity */
    CHECK(orc_f32_to_f16(1.0f + 1.0f / 2048.0f) == 0x3C00);   /* tie to even */
}

static void test_nibbles(void) {
    const int32_t w = 0x76543210;
    for (int s = 0; s < 8; ++s) CHECK(orc_nibble(w, s) == s);
    const int awq[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    for (int n = 0; n < 8; ++n) CHECK(orc_awq_slot(n) == awq[n]);
    const int32_t v = (int32_t)0xFEDCBA98u;
    for (int s = 0; s < 8; ++s) CHECK(orc_nibble(v, s) == 8 + s);
}

static void test_dequant_and_gemm(int fmt, int M, int K, int N, int G) {
    const int ng = K / G;
    const size_t qn = fmt == ORC_FMT_AWQ ? (size_t)K * N / 8 : (size_t)K / 8 * N;
    int32_t* qw = malloc(qn * 4);
    int32_t* qz = malloc((size_t)ng * N / 8 * 4);
    uint16_t* sc = malloc((size_t)ng * N * 2);
    uint16_t* x = malloc((size_t)M * K * 2);
    uint16_t* w16 = malloc((size_t)K * N * 2);
    uint16_t* wt = malloc((size_t)K * N * 2);
    uint16_t* y = malloc((size_t)M * N * 2);
    uint16_t* y2 = malloc((size_t)M * N * 2);
    float* yf = malloc((size_t)M * N * 4);
    int32_t* rows = malloc((size_t)M * 4);
    fill_words(qw, qn); fill_words(qz, (size_t)ng * N / 8); fill_scales(sc, (size_t)ng * N); fill_x(x, (size_t)M * K);
    const int32_t* z = fmt == ORC_FMT_GPTQ_SYM ? NULL : qz;
    CHECK(orc_dequant(fmt, qw, sc, z, NULL, K, N, G, 1, w16) == 0);
    CHECK(orc_dequant_transposed(fmt, qw, sc, z, NULL, K, N, G, 1, wt) == 0);
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) {
            const int q = orc_qweight_at(fmt, qw, K, N, k, n);
            const int zz = orc_zero_at(fmt, z, N, k / G, n, 1);
            const float want = (float)(q - zz) * orc_f16_to_f32(sc[(size_t)(k / G) * N + n]);
            CHECK(w16[(size_t)k * N + n] == orc_f32_to_f16(want));
            CHECK(wt[(size_t)n * K + k] == w16[(size_t)k * N + n]);
        }
    CHECK(orc_w4a16_gemm(fmt, x, qw, sc, z, NULL, M, N, K, G, 1, 1, y, yf) == 0);
    orc_gemm_f16(x, w16, M, N, K, 1, y2, NULL);
    CHECK(memcmp(y, y2, (size_t)M * N * 2) == 0);
    for (int m = 0; m < M; ++m) rows[m] = M - 1 - m;
    CHECK(orc_w4a16_gemm_rows(fmt, x, qw, sc, z, NULL, M, N, K, G, 1, rows, M, y2) == 0);
    for (int m = 0; m < M; ++m) CHECK(memcmp(y2 + (size_t)m * N, y + (size_t)(M - 1 - m) * N, (size_t)N * 2) == 0);
    /* one-hot row: y = that row of W16 */
    memset(x, 0, (size_t)M * K * 2);
    const int kk = (int)(rnd() % (uint32_t)K);
    x[kk] = 0x3C00;   /* 1.0 in row 0 */
    orc_gemm_f16(x, w16, 1, N, K, 1, y2, NULL);
    CHECK(memcmp(y2, w16 + (size_t)kk * N, (size_t)N * 2) == 0);
    /* identity g_idx equals no g_idx; out-of-range g_idx is rejected */
    int32_t* gi = malloc((size_t)K * 4);
    for (int k = 0; k < K; ++k) gi[k] = k / G;
    CHECK(orc_dequant(fmt, qw, sc, z, gi, K, N, G, 1, wt) == 0);
    CHECK(memcmp(wt, w16, (size_t)K * N * 2) == 0);
    gi[K - 1] = ng;
    CHECK(orc_dequant(fmt, qw, sc, z, gi, K, N, G, 1, wt) != 0);
    free(gi);
    if (fmt == ORC_FMT_GPTQ) {   /* qzeros of nibble 7 with +1 = the symmetric zero 8 */
        for (size_t i = 0; i < (size_t)ng * N / 8; ++i) qz[i] = 0x77777777;
        CHECK(orc_dequant(ORC_FMT_GPTQ, qw, sc, qz, NULL, K, N, G, 1, w16) == 0);
        CHECK(orc_dequant(ORC_FMT_GPTQ_SYM, qw, sc, NULL, NULL, K, N, G, 1, wt) == 0);
        CHECK(memcmp(w16, wt, (size_t)K * N * 2) == 0);
    }
    free(qw); free(qz); free(sc); free(x); free(w16); free(wt); free(y); free(y2); free(yf); free(rows);
}

static void test_moe(int T, int E, int topk, int bm) {
    float* logits = malloc((size_t)T * E * 4);
    int32_t* ids = malloc((size_t)T * topk * 4);
    float* w = malloc((size_t)T * topk * 4);
    for (int i = 0; i < T * E; ++i) logits[i] = ((float)(rnd() % 2001) - 1000.0f) / 300.0f;
    orc_moe_route(logits, T, E, topk, ids, w);
    for (int t = 0; t < T; ++t) {
        float s = 0.f;
        for (int j = 0; j < topk; ++j) { s += w[t * topk + j]; CHECK(ids[t * topk + j] >= 0 && ids[t * topk + j] < E); }
        CHECK(fabsf(s - 1.0f) < 1e-5f);
    }
    const int cap = T * topk + E * (bm - 1);
    int32_t* sorted = malloc((size_t)cap * 4);
    int32_t* experts = malloc((size_t)(cap / bm + 1) * 4);
    const int n = orc_moe_align(ids, T, topk, E, bm, sorted, experts);
    CHECK(n % bm == 0 && n <= cap);
    int* seen = calloc((size_t)T * topk, sizeof(int));
    for (int i = 0; i < n; ++i) {
        const int p = sorted[i];
        if (p == T * topk) continue;
        CHECK(p >= 0 && p < T * topk);
        if (p >= 0 && p < T * topk) { ++seen[p]; CHECK(ids[p] == experts[i / bm]); }
    }
    for (int p = 0; p < T * topk; ++p) CHECK(seen[p] == 1);
    free(logits); free(ids); free(w); free(sorted); free(experts); free(seen);
}

int main(void) {
    test_f16();
    test_nibbles();
    const int shapes[][4] = {{1, 8, 8, 8}, {3, 128, 64, 128}, {5, 256, 136, 64}, {2, 64, 8, 32}, {1, 512, 256, 512}};
    for (int f = 0; f < 3; ++f)
        for (size_t i = 0; i < sizeof shapes / sizeof shapes[0]; ++i)
            test_dequant_and_gemm(f, shapes[i][0], shapes[i][1], shapes[i][2], shapes[i][3]);
    test_moe(1, 1, 1, 1);
    test_moe(37, 8, 2, 16);
    test_moe(100, 3, 3, 64);
    for (uint32_t i = 0; i < 20000; ++i) {
        const uint16_t g = (uint16_t)rnd(), u = (uint16_t)rnd();
        (void)orc_silu_mul_f16(g, u);
    }
    if (failures) { fprintf(stderr, "%d check(s) failed\n", failures); return 1; }
    printf("orc_selftest: all checks passed\n");
    return 0;
}
