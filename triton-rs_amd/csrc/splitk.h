// Split-K hand-off shared by the GEMV and MFMA kernels: the workgroups of one output tile
// each store fp32 partial sums; a workgroup that sees every split of the tile published
// sums them in split order (deterministic) and writes fp16.
//
// The protocol avoids both whole-cache maintenance and contended atomics, which on this
// part cost more than the weight stream itself (a __threadfence() emits an L2 write-back
// and invalidate in every wave; a returning atomic on a counter shared by 16 workgroups
// serialises at ~0.25 us each):
//  1. partials are stored with agent-scope atomic stores (global_store ... sc1, written
//     through to the level all XCDs share) and the wave waits for them (vmcnt(0));
//  2. the workgroup then publishes its own flag (one word per split: no contention) the
//     same way, and waits again;
//  3. wave 0 reads all flags of the tile with agent-scope loads (sc1: not served from a
//     stale L1/L2) in one batch. The workgroup whose flag store completed last reads after
//     every other flag store completed, so at least one workgroup sees all flags set.
//     Several may: they compute and store identical values.
//  4. a finisher reads the partials (sc1), sums them in split order, stores fp16 and clears
//     the tile's flags. No flag of this call can be set after that: every split had
//     published before the finisher saw them all.
#pragma once
#include "device_common.h"

namespace w4a16 {

__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void wait_vm_stores() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores have completed
}

// Called by every thread after storing its partials with st_coherent. `flags` are the
// tile's `splits` words (zero between calls). Returns true in a finishing workgroup.
__device__ __forceinline__ bool splitk_arrive(uint32_t* flags, int split, int splits,
                                              int* lds_flag) {
    wait_vm_stores();
    __syncthreads();
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) {
            __hip_atomic_store(flags + split, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_vm_stores();
        }
        uint32_t seen = 1u;
        for (int i = threadIdx.x; i < splits; i += 64)
            seen &= __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool all = __all(seen != 0u);
        if (threadIdx.x == 0) *lds_flag = all ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

__device__ __forceinline__ void splitk_clear(uint32_t* flags, int splits) {
    for (int i = threadIdx.x; i < splits; i += blockDim.x)
        __hip_atomic_store(flags + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads of a batch of FIN_BATCH splits are all issued before the first add (addresses past
// the last split are clamped to it and their values masked): ceil(splits / FIN_BATCH)
// memory round trips per output instead of one per split.
constexpr int FIN_BATCH = 32;

__device__ __forceinline__ float sum_splits(const float* src, size_t stride, int splits) {
    float s = 0.f;
    for (int sp = 0; sp < splits; sp += FIN_BATCH) {
        float v[FIN_BATCH];
#pragma unroll
        for (int j = 0; j < FIN_BATCH; ++j)
            v[j] = ld_coherent(src + (size_t)min(sp + j, splits - 1) * stride);
#pragma unroll
        for (int j = 0; j < FIN_BATCH; ++j) s += (sp + j < splits) ? v[j] : 0.f;
    }
    return s;
}

// Finish columns [n0, n0 + C) of an [M, N] output whose partials are ws[split][M][N].
template <int M>
__device__ __forceinline__ void splitk_finish(const float* __restrict__ ws, half_t* __restrict__ out,
                                              uint32_t* flags, int splits, int N, int n0, int C) {
    const size_t stride = (size_t)M * N;
    for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
        const int m = i / C, c = i - m * C;
        const size_t off = (size_t)m * N + n0 + c;
        out[off] = (half_t)sum_splits(ws + off, stride, splits);
    }
    splitk_clear(flags, splits);
}

// Runtime-row variant: rows [m0, m0 + rows) of an [M, N] output.
__device__ __forceinline__ void splitk_finish_rows(const float* __restrict__ ws,
                                                   half_t* __restrict__ out, uint32_t* flags,
                                                   int splits, int M, int N, int m0, int rows,
                                                   int n0, int C) {
    const size_t stride = (size_t)M * N;
    for (int i = threadIdx.x; i < rows * C; i += blockDim.x) {
        const int r = i / C, c = i - r * C;
        const size_t off = (size_t)(m0 + r) * N + n0 + c;
        out[off] = (half_t)sum_splits(ws + off, stride, splits);
    }
    splitk_clear(flags, splits);
}

}  // namespace w4a16
