// Launchers for the generic strided GEMM (strided_body.h) and the standalone dequant kernels.
#include <type_traits>

#include "strided_body.h"

namespace w4a16 {

template <int FMT, typename E>
__global__ void __launch_bounds__(256) strided_gemm_kernel(StridedParams p) {
    strided_gemm_body<FMT, E>(p);
}

// A gated launch is a fallback that usually exits at once (the act-order route runs it
// behind the tiled prefill, for a g_idx that route cannot take): launching one workgroup per
// tile would cost about 4 us of empty workgroups at M = 2048, N = 6144, so it gets at most
// STR_GATED_GRID workgroups that walk the tiles.
constexpr int STR_GATED_GRID = 512;

template <typename E>
static void launch_strided_e(int fmt, const StridedParams& p, hipStream_t st) {
    const int tm = (p.m + STR_BM - 1) / STR_BM, tn = (p.n + STR_BN - 1) / STR_BN;
    const dim3 grid = p.gate && (int64_t)tm * tn > STR_GATED_GRID ? dim3(STR_GATED_GRID) : dim3(tm, tn);
    const dim3 block(256);
    if (fmt == FMT_AWQ) hipLaunchKernelGGL((strided_gemm_kernel<FMT_AWQ, E>), grid, block, 0, st, p);
    else if (fmt == FMT_GPTQ) hipLaunchKernelGGL((strided_gemm_kernel<FMT_GPTQ, E>), grid, block, 0, st, p);
    else if (fmt == FMT_GPTQ_SYM) hipLaunchKernelGGL((strided_gemm_kernel<FMT_GPTQ_SYM, E>), grid, block, 0, st, p);
    else if constexpr (std::is_same<E, half_t>::value)   // prepared layout: fp16 only
        hipLaunchKernelGGL((strided_gemm_kernel<FMT_PREP, E>), grid, block, 0, st, p);
}

hipError_t launch_strided_gemm(int fmt, const StridedParams& p, hipStream_t st, bool bf16) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (bf16) launch_strided_e<bf16_t>(fmt, p, st);
    else launch_strided_e<half_t>(fmt, p, st);
    return hipGetLastError();
}

// ------------------------------------------------------------------ dequant

// One thread per packed word. GPTQ word (kp, n) -> 8 consecutive k of column n;
// AWQ word (k, wn) -> 8 consecutive columns of row k. E: fp16 or bfloat16 scales and output.
template <int FMT, typename E>
__global__ void __launch_bounds__(256) dequant_kernel(DequantParams p) {
    typedef typename vec8<E>::type e8_t;
    const E* scales = reinterpret_cast<const E*>(p.scales);
    E* out = reinterpret_cast<E*>(p.out);
    const int64_t NW = (FMT == FMT_AWQ) ? (p.N >> 3) : p.N;
    const int64_t rows = (FMT == FMT_AWQ) ? p.K : (p.K >> 3);
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * NW) return;
    const int64_t r = idx / NW, c = idx - r * NW;
    const uint32_t word = p.qweight[idx];
    E v[8];
    if constexpr (FMT == FMT_AWQ) {
        const int k = (int)r;
        const int g = p.g_idx ? min(max(p.g_idx[k], 0), p.K / p.G - 1) : k / p.G;
        const uint32_t qz = p.qzeros[(int64_t)g * NW + c];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = (int)(8 * c + j);
            v[j] = dequant1(nib(word, awq_slot(n)), zero_of<FMT>(qz, n, 0),
                            scales[(int64_t)g * p.N + n]);
        }
        if (!p.transposed) {
            *reinterpret_cast<e8_t*>(out + (int64_t)k * p.N + 8 * c) =
                e8_t{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) out[(8 * c + j) * p.K + k] = v[j];
        }
    } else {
        const int n = (int)c;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = (int)(8 * r + j);
            const int g = p.g_idx ? min(max(p.g_idx[k], 0), p.K / p.G - 1) : k / p.G;
            uint32_t qz = 0;
            if constexpr (FMT == FMT_GPTQ) qz = p.qzeros[(int64_t)g * (p.N >> 3) + (n >> 3)];
            v[j] = dequant1(nib(word, j), zero_of<FMT>(qz, n, p.zero_offset),
                            scales[(int64_t)g * p.N + n]);
        }
        if (p.transposed) {
            *reinterpret_cast<e8_t*>(out + (int64_t)n * p.K + 8 * r) =
                e8_t{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) out[(8 * r + j) * p.N + n] = v[j];
        }
    }
}

template <typename E>
static void launch_dequant_e(int fmt, const DequantParams& p, hipStream_t st) {
    const int64_t words = (int64_t)p.K * p.N / 8;
    const dim3 grid((unsigned)((words + 255) / 256)), block(256);
    if (fmt == FMT_AWQ) hipLaunchKernelGGL((dequant_kernel<FMT_AWQ, E>), grid, block, 0, st, p);
    else if (fmt == FMT_GPTQ) hipLaunchKernelGGL((dequant_kernel<FMT_GPTQ, E>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((dequant_kernel<FMT_GPTQ_SYM, E>), grid, block, 0, st, p);
}

hipError_t launch_dequant(int fmt, const DequantParams& p, hipStream_t st, bool bf16) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (bf16) launch_dequant_e<bf16_t>(fmt, p, st);
    else launch_dequant_e<half_t>(fmt, p, st);
    return hipGetLastError();
}

}  // namespace w4a16
