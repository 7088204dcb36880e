// The C-ABI op layer (api.cpp, hiprt.cpp) under AddressSanitizer and UndefinedBehaviorSanitizer:
// every entry point's argument validation (which runs before any HIP call, so no GPU is
// needed) and the kernel planners over a sweep of shapes up to the int32 limits, where the
// size arithmetic (tile counts, split counts, workspace sizes) must not overflow.
// Exit status 0 = all passed.
#include <climits>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "w4a16.h"

static int failures = 0;
#define CHECK(c) do { if (!(c)) { std::fprintf(stderr, "FAIL %s:%d: %s (%s)\n", __FILE__, __LINE__, #c, w4a16_last_error()); ++failures; } } while (0)

int main() {
    void* v = reinterpret_cast<void*>(uintptr_t(256));
    int32_t* vi = static_cast<int32_t*>(v);
    // ---- w4a16_gemm / noalloc / act-order validation
    for (auto fn : {w4a16_gemm, w4a16_gemm_noalloc}) {
        CHECK(fn(nullptr, 7, v, v, v, v, nullptr, v, 1, 4096, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_AWQ, nullptr, v, v, v, nullptr, v, 1, 4096, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_GPTQ, v, v, v, nullptr, nullptr, v, 1, 4096, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_AWQ, v, v, v, v, nullptr, v, 0, 4096, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_AWQ, v, v, v, v, nullptr, v, 1, 4100, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_AWQ, v, v, v, v, nullptr, v, 1, 4096, 4000, 128, 1) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_GPTQ, v, v, v, v, nullptr, v, 1, 4096, 4096, 128, 99) == W4A16_ERR_INVALID_ARG);
        CHECK(fn(nullptr, W4A16_FMT_GPTQ, v, v, v, v, nullptr, v, INT_MIN, INT_MIN, INT_MIN, INT_MIN, 1) == W4A16_ERR_INVALID_ARG);
    }
    CHECK(w4a16_prepare_act_order(nullptr, W4A16_FMT_AWQ, v, vi, 4096, 512, 128, vi, vi) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_prepare_act_order(nullptr, W4A16_FMT_GPTQ, v, vi, 4096, 512, 128, v, vi) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_prepare_act_order(nullptr, W4A16_FMT_GPTQ, v, vi, 8 * 70000, 512, 128, vi + 64, vi) == W4A16_ERR_INVALID_ARG ||
          w4a16_prepare_act_order(nullptr, W4A16_FMT_GPTQ, v, vi, 8 * 70000, 512, 128, vi + 64, vi) == W4A16_ERR_UNSUPPORTED);
    CHECK(w4a16_gemm_act_order(nullptr, W4A16_FMT_GPTQ, v, v, v, v, nullptr, v, 1, 512, 4096, 128, 1) == W4A16_ERR_INVALID_ARG);
    // ---- reference-named entry points
    CHECK(w4a16_gptq_gemm_typed(nullptr, nullptr, v, v, v, v, 1, 64, 64, 64, 64, 1, 64, 1, 64, 1, 8, 1, 64, 1) == W4A16_ERR_INVALID_ARG);
    CHECK(awq_gemm_int4_typed(nullptr, v, v, v, v, v, -1, 64, 64, 64, 64, 1, 8, 1, 64, 1, 8, 1, 64, 1) == W4A16_ERR_INVALID_ARG);
    CHECK(awq_gemm_int4_typed(nullptr, v, v, v, v, v, 0, 64, 64, 64, 64, 1, 8, 1, 64, 1, 8, 1, 64, 1) == W4A16_OK);
    CHECK(dequant_int4_to_fp16(nullptr, vi, v, vi, v, 256, 64, 128, 9) == W4A16_ERR_INVALID_ARG);
    CHECK(dequant_int4_sym_to_fp16(nullptr, nullptr, v, v, 256, 64, 128) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_dequant(nullptr, W4A16_FMT_AWQ, v, v, v, nullptr, v, 256, 60, 128, 0, 0) == W4A16_ERR_INVALID_ARG);
    // ---- MoE validation
    CHECK(w4a16_moe_route(nullptr, nullptr, 4, 8, 2, 1, vi, static_cast<float*>(v)) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_moe_route(nullptr, static_cast<float*>(v), 4, 300, 2, 1, vi, static_cast<float*>(v)) == W4A16_ERR_UNSUPPORTED);
    CHECK(w4a16_moe_align(nullptr, vi, 1024, 8, 64, 1024, vi, vi, vi) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_moe_align(nullptr, vi, INT_MAX, INT_MAX, INT_MAX, INT_MAX, vi, vi, vi) != W4A16_OK);
    CHECK(w4a16_moe_gemm(nullptr, 0, v, 2, v, v, v, 0, 0, 0, 8, vi, vi, vi, v, 1024, 1004, 4096, 128, 64, 1536, 1) == W4A16_ERR_INVALID_ARG);
    CHECK(w4a16_moe_gemm(nullptr, 0, v, 2, v, v, v, 0, 0, 0, 0, vi, vi, vi, v, 1024, 1024, 4096, 128, 64, 1536, 1) == W4A16_ERR_INVALID_ARG);
    CHECK(fused_silu_mul_interleaved_f16(nullptr, v, v, 0, 10) == W4A16_ERR_INVALID_ARG);
    CHECK(fused_silu_mul_interleaved_f16(nullptr, v, v, 10, 0) == W4A16_OK);
    CHECK(w4a16_moe_sum(nullptr, v, static_cast<float*>(v), v, 4, 2, 12) == W4A16_ERR_INVALID_ARG);
    // workspace sizes: monotone in T, and zero for invalid shapes
    size_t prev = 0;
    for (int T = 1; T <= 1 << 16; T *= 4) {
        const size_t ws = w4a16_fused_moe_workspace_size(T, 8, 2, 14336, 4096, 64);
        CHECK(ws > prev);
        prev = ws;
    }
    CHECK(w4a16_fused_moe_workspace_size(0, 8, 2, 14336, 4096, 64) == 0);
    CHECK(w4a16_fused_moe(nullptr, 0, v, static_cast<float*>(v), 512, 4096, 14336, 8, 2, 1, v, v, v, v, v, v,
                          128, 64, 1, v, 1, v) == W4A16_ERR_INVALID_ARG);
    // ---- planners over a shape sweep (host arithmetic only)
    const int Ms[] = {1, 2, 3, 4, 5, 8, 9, 16, 33, 64, 65, 128, 255, 2048, 65536, 1 << 20};
    const int Ns[] = {8, 64, 136, 256, 4096, 6144, 14336, 1 << 20, (INT_MAX / 256) * 8};
    const int Ks[] = {8, 64, 128, 1024, 4096, 14336, 1 << 20};
    int plans = 0;
    for (int fmt = 0; fmt < 3; ++fmt)
        for (int M : Ms)
            for (int N : Ns)
                for (int K : Ks)
                    for (int G : {32, 128}) {
                        if (K % G) continue;
                        int kernel = 0;
                        const int rc = w4a16_gemm_plan(fmt, M, N, K, G, fmt == 0 && M <= 64, &kernel);
                        CHECK(rc == W4A16_OK);
                        CHECK(kernel >= W4A16_KERNEL_GEMV && kernel <= W4A16_KERNEL_STRIDED);
                        if (fmt != 1) {
                            const int qwk = fmt == 2 ? N / 8 : N;
                            const int32_t st[10] = {K, 1, qwk, 1, N, 1, N / 8, 1, N, 1};
                            int tk = 0;
                            CHECK(w4a16_typed_plan(fmt, M, N, K, G, st, 1, &tk) == W4A16_OK);
                            CHECK(tk == kernel || (fmt == 0 && M <= 64 && tk != 0));
                        }
                        ++plans;
                    }
    CHECK(plans > 1000);
    // ---- runtime shim without a usable device (CPU build) or with one: argument checks
    hiprt_ctx* ctx = nullptr;
    CHECK(hiprt_create(0, nullptr) == W4A16_ERR_INVALID_ARG);
    CHECK(hiprt_module_load(nullptr, v, 16, nullptr) == W4A16_ERR_INVALID_ARG);
    CHECK(hiprt_launch(nullptr, nullptr, "k", nullptr, nullptr, 0, nullptr, nullptr, 0) == W4A16_ERR_INVALID_ARG);
    CHECK(hiprt_destroy(nullptr) == W4A16_ERR_INVALID_ARG);
    (void)ctx;
    CHECK(std::strstr(w4a16_version(), "gfx950") != nullptr);
    if (failures) { std::fprintf(stderr, "%d check(s) failed\n", failures); return 1; }
    std::printf("abi_selftest: all checks passed (%d plans)\n", plans);
    return 0;
}
