// Split-K hand-off shared by the GEMV and MFMA kernels: the workgroups of one output tile
// each store fp32 partial sums; a workgroup that sees every split of the tile published
// sums them in a fixed order (deterministic) and writes fp16.
//
// The protocol avoids both whole-cache maintenance and contended atomics, which on this
// part cost more than the weight stream itself (a __threadfence() emits an L2 write-back
// and invalidate in every wave; a returning atomic on a counter shared by 16 workgroups
// serialises at ~0.25 us each):
//  1. partials are stored with agent-scope atomic stores (global_store ... sc1, written
//     through to the level all XCDs share) and the wave waits for them (vmcnt(0));
//  2. the workgroup then publishes its own flag the same way, and waits again. Each flag
//     has a 256-byte line of its own: with a tile's flags packed in one line, every flag
//     store and load of the tile queues at the same memory channel;
//  3. wave 0 reads all flags of the tile with agent-scope loads (sc1: not served from a
//     stale L1/L2) in one batch. The workgroup whose flag store completed last reads after
//     every other flag store completed, so at least one workgroup sees all flags set.
//     Several may: they compute and store identical values.
//  4. a finisher reads the partials (sc1), sums them in a fixed order, stores fp16 and
//     clears the tile's flags. No flag of this call can be set after that: every split had
//     published before the finisher saw them all.
#pragma once
#include "device_common.h"
#include "launch.h"

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

// The flags of a tile (FLAG_STRIDE words apart, launch.h).
__device__ __forceinline__ uint32_t* splitk_flags(uint32_t* base, int tile, int splits) {
    return base + (size_t)tile * splits * FLAG_STRIDE;
}

// Called by every thread after storing its partials with st_coherent. `flags` are the
// tile's `splits` flags (zero between calls). Returns true in a finishing workgroup.
__device__ __forceinline__ bool splitk_arrive(uint32_t* flags, int split, int splits,
                                              int* lds_flag) {
    wait_vm_stores();
    __syncthreads();
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) {
            __hip_atomic_store(flags + (size_t)split * FLAG_STRIDE, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            wait_vm_stores();
        }
        uint32_t seen = 1u;
        for (int i = threadIdx.x; i < splits; i += 64)
            seen &= __hip_atomic_load(flags + (size_t)i * FLAG_STRIDE, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
        const bool all = __all(seen != 0u);
        if (threadIdx.x == 0) *lds_flag = all ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

__device__ __forceinline__ void splitk_clear(uint32_t* flags, int splits) {
    for (int i = threadIdx.x; i < splits; i += blockDim.x)
        __hip_atomic_store(flags + (size_t)i * FLAG_STRIDE, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Four partials (16-byte aligned) as two 64-bit agent-scope loads.
__device__ __forceinline__ float4_t ld_coherent4(const float* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return float4_t{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                    __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32))};
}

// Finish columns [n0, n0 + C) of rows [m0, m0 + rows) of an [M, N] output whose partials
// are ws[split][M][N] (C % 4 == 0, N % 4 == 0). Work is cut into float4 column chunks;
// when a workgroup has more threads than chunks, the splits are divided into groups summed
// by different threads and combined through LDS. Each thread issues the loads of a batch
// of up to FB splits before its first add, so a chunk costs ceil(splits / groups / FB)
// memory round trips. Summation order: splits in order within a group, groups in order.
constexpr int FB = 16;
constexpr int FINISH_MAX_THREADS = 512;

__device__ __forceinline__ void splitk_finish_rows(const float* __restrict__ ws,
                                                   half_t* __restrict__ out, uint32_t* flags,
                                                   int splits, int M, int N, int m0, int rows,
                                                   int n0, int C) {
    __shared__ float4_t part[FINISH_MAX_THREADS];
    const int T = blockDim.x;   // <= FINISH_MAX_THREADS
    const int cpr = C / 4;                       // chunks per row
    const int chunks = rows * cpr;
    const int groups = chunks >= T ? 1 : min(splits, T / chunks);
    const int per = (splits + groups - 1) / groups;
    const size_t stride = (size_t)M * N;
    const int span = groups == 1 ? T : chunks;   // chunks handled per pass
    for (int c0 = 0; c0 < chunks; c0 += span) {
        const int ch = c0 + (int)threadIdx.x % span;
        const int gi = (int)threadIdx.x / span;
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        size_t off = 0;
        if (ch < chunks && gi < groups) {
            const int r = ch / cpr, c = ch - r * cpr;
            off = (size_t)(m0 + r) * N + n0 + 4 * c;
            const int s0 = gi * per, s1 = min(splits, s0 + per);
            for (int sb = s0; sb < s1; sb += FB) {
                float4_t v[FB];
#pragma unroll
                for (int t = 0; t < FB; ++t)
                    if (sb + t < s1) v[t] = ld_coherent4(ws + (size_t)(sb + t) * stride + off);
#pragma unroll
                for (int t = 0; t < FB; ++t)
                    if (sb + t < s1) acc += v[t];
            }
        }
        if (groups > 1) {
            part[threadIdx.x] = acc;
            __syncthreads();
            if (gi == 0 && ch < chunks) {
                for (int g = 1; g < groups; ++g) acc += part[g * span + threadIdx.x];
            }
            __syncthreads();
        }
        if (gi == 0 && ch < chunks) {
            const half2_t lo = {(half_t)acc[0], (half_t)acc[1]};
            const half2_t hi = {(half_t)acc[2], (half_t)acc[3]};
            *reinterpret_cast<u32x2*>(out + off) = u32x2{as_u32(lo), as_u32(hi)};
        }
    }
    splitk_clear(flags, splits);
}

template <int M>
__device__ __forceinline__ void splitk_finish(const float* __restrict__ ws, half_t* __restrict__ out,
                                              uint32_t* flags, int splits, int N, int n0, int C) {
    splitk_finish_rows(ws, out, flags, splits, M, N, 0, M, n0, C);
}

}  // namespace w4a16
