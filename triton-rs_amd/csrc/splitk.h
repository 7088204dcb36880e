// Split-K fix-up shared by the GEMV and MFMA kernels: each workgroup of a column tile
// stores its fp32 partial sums, and the last one to arrive sums them in split order
// (deterministic) and writes fp16.
#pragma once
#include "device_common.h"

namespace w4a16 {

// Split-K hand-off without whole-cache maintenance. Partials are written with agent-scope
// atomic stores (global_store ... sc1: written through to the level shared by all XCDs) and
// read back with agent-scope atomic loads (sc1: never served from a possibly stale L1/L2), so
// no L2 write-back (buffer_wbl2) or invalidate (buffer_inv) is needed; a __threadfence()
// here would emit both in every wave.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of the block after it has stored its partials (st_coherent).
// Returns true in the (single) block that must produce the final output for the tile.
__device__ __forceinline__ bool splitk_arrive(uint32_t* counter, int splits, int* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = (prev == (uint32_t)(splits - 1));
    }
    __syncthreads();
    return *lds_flag != 0;
}

__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum the partials of one column tile in split order and store fp16; reset the counter.
// The loads of a batch of FIN_BATCH splits are all issued before the first add (addresses
// past the last split are clamped to it and their values masked), so a tile costs
// ceil(splits / FIN_BATCH) memory round trips instead of one per split.
constexpr int FIN_BATCH = 32;

template <int M>
__device__ __forceinline__ void splitk_finish(const float* __restrict__ ws, half_t* __restrict__ out,
                                              uint32_t* counter, int splits, int N, int n0,
                                              int C) {
    const size_t stride = (size_t)M * N;
    for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
        const int m = i / C, c = i - m * C;
        const size_t off = (size_t)m * N + n0 + c;
        const float* src = ws + off;
        float s = 0.f;
        for (int sp = 0; sp < splits; sp += FIN_BATCH) {
            float v[FIN_BATCH];
#pragma unroll
            for (int j = 0; j < FIN_BATCH; ++j)
                v[j] = ld_coherent(src + (size_t)min(sp + j, splits - 1) * stride);
#pragma unroll
            for (int j = 0; j < FIN_BATCH; ++j) s += (sp + j < splits) ? v[j] : 0.f;
        }
        out[off] = (half_t)s;
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Runtime-row variant for the MFMA kernels: rows [m0, m0 + rows) of an [M, N] output.
__device__ __forceinline__ void splitk_finish_rows(const float* __restrict__ ws,
                                                   half_t* __restrict__ out, uint32_t* counter,
                                                   int splits, int M, int N, int m0, int rows,
                                                   int n0, int C) {
    const size_t stride = (size_t)M * N;
    for (int i = threadIdx.x; i < rows * C; i += blockDim.x) {
        const int r = i / C, c = i - r * C;
        const size_t off = (size_t)(m0 + r) * N + n0 + c;
        const float* src = ws + off;
        float s = 0.f;
        for (int sp = 0; sp < splits; sp += FIN_BATCH) {
            float v[FIN_BATCH];
#pragma unroll
            for (int j = 0; j < FIN_BATCH; ++j)
                v[j] = ld_coherent(src + (size_t)min(sp + j, splits - 1) * stride);
#pragma unroll
            for (int j = 0; j < FIN_BATCH; ++j) s += (sp + j < splits) ? v[j] : 0.f;
        }
        out[off] = (half_t)s;
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace w4a16
