// Split-K hand-off shared by the GEMV and small-batch MFMA kernels: the workgroups of one
// output tile each store fp32 partial sums; the workgroup that arrives last sums them in a
// fixed order (deterministic) and writes fp16.
//
// Protocol (one 32-bit counter per tile, zero between calls):
//  1. every thread stores its partials, and the workgroup waits until they have completed
//     (s_waitcnt vmcnt(0): the stores are acknowledged by the level named below);
//  2. one thread adds 1 to the tile's counter with a returning atomic (performed at L2, the
//     same instruction at every scope on this target). The workgroup that reads
//     `splits - 1` arrived last: every other split had completed its stores before its own
//     add, so all partials are visible to it. It resets the counter to 0 for the next call;
//  3. the last workgroup reads the partials, sums them in split order and stores fp16.
//
// Where the partials live (template parameter SC):
//  * SCOPE_DEVICE: stores and loads at agent scope (global_store/load ... sc1), coherent
//    between the XCDs' L2 caches. Works for any workgroup placement.
//  * SCOPE_XCD: stores and loads at workgroup scope (sc0: past the CU's L1, coherent in its
//    XCD's L2). Correct only when every split of a tile runs on the same XCD. The
//    dispatcher hands workgroup b of a launch to XCD b mod 8 (checked once per device at
//    run time, api.cpp); the kernels using this mode give all splits of a tile block ids
//    that are congruent mod 8. The hand-off then never leaves the L2: measured on the
//    AWQ GEMV (K=4096, N=14336) 9.2 us per call against 10.4 us for a device-scope flag
//    protocol, with the same kernels.
//
// A __threadfence() is not used: on this part it emits an L2 write-back and invalidate in
// every wave, which costs more than the weight stream itself.
#pragma once
#include "device_common.h"
#include "launch.h"

namespace w4a16 {

constexpr int SCOPE_DEVICE = __HIP_MEMORY_SCOPE_AGENT;
constexpr int SCOPE_XCD = __HIP_MEMORY_SCOPE_WORKGROUP;

template <int SC>
__device__ __forceinline__ void st_partial(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, SC);
}

// Four partials (16-byte aligned) as two 64-bit loads at scope SC.
template <int SC>
__device__ __forceinline__ float4_t ld_partial4(const float* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, SC);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, SC);
    return float4_t{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                    __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32))};
}

__device__ __forceinline__ void wait_vm_stores() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores have completed
}

// The counter of a tile (FLAG_STRIDE words apart: a 256-byte line each, launch.h).
__device__ __forceinline__ uint32_t* splitk_counter(uint32_t* base, int tile) {
    return base + (size_t)tile * FLAG_STRIDE;
}

// Called by every thread after storing its partials with st_partial. Returns true in the
// workgroup that arrived last.
__device__ __forceinline__ bool splitk_arrive(uint32_t* counter, int splits, int* lds_flag) {
    wait_vm_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t before =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before == (uint32_t)splits - 1u;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// Workgroup-id -> (tile, split). XCD mode: a 1-D grid of tiles * splits workgroups; XCD
// c = b mod 8 owns tiles [c * T/8, (c+1) * T/8) with all their splits, neighbouring tiles
// on one XCD (they share DRAM pages through its L2: the 128-byte-per-row weight stream
// of the GEMV reads as fast as 256-byte rows this way). Requires tiles % 8 == 0.
// Otherwise: blockIdx.x = tile, blockIdx.y = split.
template <bool XCD>
__device__ __forceinline__ void tile_of_block(int tiles, int splits, int& tile, int& split) {
    if constexpr (XCD) {
        const int b = blockIdx.x, c = b & 7, u = b >> 3;
        const int t = u / splits;
        tile = c * (tiles >> 3) + t;
        split = u - t * splits;
    } else {
        tile = blockIdx.x;
        split = blockIdx.y;
    }
}

// Finish columns [n0, n0 + C) of rows [m0, m0 + rows) of an [M, N] output whose partials
// are ws[split][M][N]. Two layouts of the work, chosen by size:
//  * at most one entry (row, column) per thread: a thread sums its entry's partials with
//    scalar loads, FB in flight before the first add (a remainder of fewer than FB splits
//    in batches of FB/4); spare threads take groups of splits, combined through LDS;
//  * more entries than threads: float4 column chunks (C % 4 == 0, N % 4 == 0), up to FB4
//    splits in flight per chunk (two chunks at a time when there are at least two per thread
//    and at most FB4/2 splits), groups of splits when threads outnumber chunks.
// Summation order: splits in order within a group, groups in order.
constexpr int FB = 16;
constexpr int FB4 = 16;
constexpr int FINISH_MAX_THREADS = 512;

// E: the output element (fp16, or bf16 for the bfloat16 instantiations).
template <int SC, typename E = half_t>
__device__ __forceinline__ void splitk_finish_rows(const float* __restrict__ ws,
                                                   E* __restrict__ out, int splits, int M,
                                                   int N, int m0, int rows, int n0, int C) {
    __shared__ float4_t part[FINISH_MAX_THREADS];
    const int T = blockDim.x;   // <= FINISH_MAX_THREADS
    const size_t stride = (size_t)M * N;
    if (rows * C <= T) {
        const int entries = rows * C;
        const int groups = min(splits, T / entries);
        const int per = (splits + groups - 1) / groups;
        const int e = (int)threadIdx.x % entries, gi = (int)threadIdx.x / entries;
        const int r = e / C, c = e - r * C;
        const size_t off = (size_t)(m0 + r) * N + n0 + c;
        float acc = 0.f;
        if (gi < groups) {
            const int s0 = gi * per, s1 = min(splits, s0 + per);
            int sb = s0;
            for (; sb + FB <= s1; sb += FB) {   // full batches: loads without conditions
                float v[FB];
#pragma unroll
                for (int t = 0; t < FB; ++t)
                    v[t] = __hip_atomic_load(ws + (size_t)(sb + t) * stride + off, __ATOMIC_RELAXED, SC);
#pragma unroll
                for (int t = 0; t < FB; ++t) acc += v[t];
            }
            for (; sb < s1; sb += FB / 4) {
                float v[FB / 4];
#pragma unroll
                for (int t = 0; t < FB / 4; ++t)
                    v[t] = sb + t < s1 ? __hip_atomic_load(ws + (size_t)(sb + t) * stride + off,
                                                           __ATOMIC_RELAXED, SC)
                                       : 0.f;
#pragma unroll
                for (int t = 0; t < FB / 4; ++t) acc += v[t];
            }
        }
        if (groups > 1) {
            reinterpret_cast<float*>(part)[threadIdx.x] = acc;
            __syncthreads();
            if (gi == 0)
                for (int g = 1; g < groups; ++g) acc += reinterpret_cast<float*>(part)[g * entries + e];
        }
        if (gi == 0) out[off] = (E)acc;
        return;
    }
    const int cpr = C / 4;                       // chunks per row
    const int chunks = rows * cpr;
    const int groups = chunks >= T ? 1 : min(splits, T / chunks);
    const int per = (splits + groups - 1) / groups;
    const int span = groups == 1 ? T : chunks;   // chunks handled per pass
    if (groups == 1 && chunks >= 2 * T && splits <= FB4 / 2) {
        // two chunks per thread per batch: the loads of both are in flight together
        for (int c0 = 0; c0 < chunks; c0 += 2 * T) {
            const int cha = c0 + (int)threadIdx.x, chb = cha + T;
            const bool okb = chb < chunks;
            const size_t offa = (size_t)(m0 + cha / cpr) * N + n0 + 4 * (cha % cpr);
            const size_t offb = okb ? (size_t)(m0 + chb / cpr) * N + n0 + 4 * (chb % cpr) : offa;
            float4_t va[FB4 / 2], vb[FB4 / 2];
#pragma unroll
            for (int t = 0; t < FB4 / 2; ++t)
                if (t < splits) {
                    va[t] = ld_partial4<SC>(ws + (size_t)t * stride + offa);
                    vb[t] = ld_partial4<SC>(ws + (size_t)t * stride + offb);
                }
            float4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < FB4 / 2; ++t)
                if (t < splits) { a += va[t]; b += vb[t]; }
            *reinterpret_cast<u32x2*>(out + offa) = u32x2{pack2(E{}, a[0], a[1]), pack2(E{}, a[2], a[3])};
            if (okb)
                *reinterpret_cast<u32x2*>(out + offb) = u32x2{pack2(E{}, b[0], b[1]), pack2(E{}, b[2], b[3])};
        }
        return;
    }
    for (int c0 = 0; c0 < chunks; c0 += span) {
        const int ch = c0 + (int)threadIdx.x % span;
        const int gi = (int)threadIdx.x / span;
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        size_t off = 0;
        if (ch < chunks && gi < groups) {
            const int r = ch / cpr, c = ch - r * cpr;
            off = (size_t)(m0 + r) * N + n0 + 4 * c;
            const int s0 = gi * per, s1 = min(splits, s0 + per);
            for (int sb = s0; sb < s1; sb += FB4) {
                float4_t v[FB4];
#pragma unroll
                for (int t = 0; t < FB4; ++t)
                    if (sb + t < s1) v[t] = ld_partial4<SC>(ws + (size_t)(sb + t) * stride + off);
#pragma unroll
                for (int t = 0; t < FB4; ++t)
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
        if (gi == 0 && ch < chunks)
            *reinterpret_cast<u32x2*>(out + off) = u32x2{pack2(E{}, acc[0], acc[1]), pack2(E{}, acc[2], acc[3])};
    }
}

template <int M, int SC, typename E = half_t>
__device__ __forceinline__ void splitk_finish(const float* __restrict__ ws, E* __restrict__ out,
                                              int splits, int N, int n0, int C) {
    splitk_finish_rows<SC, E>(ws, out, splits, M, N, 0, M, n0, C);
}

// ------------------------------------------------------------------ fixed-point hand-off
//
// One returning 64-bit atomic add per output entry and split replaces "store partials,
// wait, count, reload": the entry's slot word carries the arrival count and an exact
// fixed-point sum, so the split whose add returns count splits - 1 holds the whole sum
// and writes the fp16 output itself (two L2 round trips instead of four; the GEMV at
// M = 1, K = 4096, N = 14336: 8.87 -> 8.51 us). Integer addition is associative, so the
// result does not depend on arrival order: repeated calls are bit-identical.
//
// Slot word (uint64, zero between calls; the last arrival stores zero back):
//   bits 58..62  arrivals A          (splits <= FIX_MAX_SPLITS)
//   bits 53..57  overflow arrivals O
//   bits  0..52  sum S of the partials in units of 2^-32, two's complement, |S| < 2^52
// Each split adds 2^58 + round(v * 2^32). Decoding old + 2^52 gives A, O and S + 2^52 with
// no carries between the fields, since 0 <= S + 2^52 < 2^53.
//
// Precision: each partial is rounded to 2^-33 (absolute), so the sum is within
// splits * 2^-33 < 2^-28 of the exact sum of the fp32 partials: below a sixteenth of the
// smallest fp16 step (2^-24) at every output magnitude.
//
// Range: partials with |v| >= 2^15, and NaN or infinity, take the fp32 path instead: the
// split stores v in the fp32 partial buffer, sets bit `split` of the entry's mask word
// (zero between calls), waits for both to complete, and adds 2^58 + 2^53. The last arrival
// then adds the flagged partials, in split order, to the fixed-point part (converted to
// fp32), and clears the mask. So every input the fp32 accumulation handles is handled, in
// a fixed order.
// (FIX_MAX_SPLITS, FIX_MAX_ENTRIES and the slot area's place are in launch.h.)
constexpr float FIX_LIMIT = 32768.0f;                            // 2^15
constexpr uint64_t FIX_ARRIVE = 1ull << 58, FIX_OVER = 1ull << 53, FIX_BIAS = 1ull << 52;

// Entries off[0..n) of an [M, N] output (mn = M * N entries) held by this thread, with
// this split's fp32 partials v[0..n), n <= E. ws is the fp32 partial buffer [splits][M][N]
// (used only for out-of-range partials). All adds are issued before the first result is
// used, so a thread's entries cost one round trip together.
// T: the output element (fp16 or bf16).
template <int SC, int E, typename T = half_t>
__device__ __forceinline__ void splitk_fixed_commit(uint64_t* __restrict__ slots,
                                                    uint32_t* __restrict__ masks,
                                                    float* __restrict__ ws, size_t mn,
                                                    T* __restrict__ out,
                                                    const size_t (&off)[E], const float (&v)[E],
                                                    int n, int split, int splits) {
    uint64_t add[E], old[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (e >= n) break;
        if (__builtin_fabsf(v[e]) < FIX_LIMIT) {   // false for NaN and infinity
            add[e] = FIX_ARRIVE + (uint64_t)(int64_t)__builtin_rintf(v[e] * 4294967296.0f);
        } else {
            st_partial<SC>(ws + (size_t)split * mn + off[e], v[e]);
            __hip_atomic_fetch_or(masks + off[e], 1u << split, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            wait_vm_stores();  // the partial and the mask bit have completed before the add
            add[e] = FIX_ARRIVE + FIX_OVER;
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (e >= n) break;
        old[e] = __hip_atomic_fetch_add(slots + off[e], add[e], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (e >= n) break;
        if (((old[e] + FIX_BIAS) >> 58) != (uint64_t)(splits - 1)) continue;
        const uint64_t u = old[e] + add[e] + FIX_BIAS;
        const int64_t sum = (int64_t)(u & ((1ull << 53) - 1)) - (int64_t)FIX_BIAS;
        float r = (float)((double)sum * (1.0 / 4294967296.0));
        if ((u >> 53) & 31u) {
            const uint32_t bits =
                __hip_atomic_load(masks + off[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int s = 0; s < splits; ++s)
                if ((bits >> s) & 1u)
                    r += s == split ? v[e]
                                    : __hip_atomic_load(ws + (size_t)s * mn + off[e], __ATOMIC_RELAXED, SC);
            __hip_atomic_store(masks + off[e], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        out[off[e]] = (T)r;
        __hip_atomic_store(slots + off[e], (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace w4a16
