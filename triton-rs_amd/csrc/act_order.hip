// GPTQ act-order (desc_act) in group order: the one-time repack of a checkpoint's qweight
// rows into the order of their groups, and the per-call gather of the activations' columns
// into the same order.
//
// A desc_act checkpoint stores row k of W in its natural place and assigns it group g_idx[k]
// (the reference has no act-order; its GEMM uses group k / G, w4a16_gptq_gemm_typed.rs:221).
// With perm the stable sort of the rows by group (perm[j] = the j-th row in group order) and
// every group holding exactly G rows, row j of the repacked matrix W'[j] = W[perm[j]] lies
// in group j / G, so
//     y = x @ W = sum_k x[:, k] W[k] = sum_j x[:, perm[j]] W'[j] = x' @ W',  x' = x[:, perm]
// and W' is an ordinary (non-act-order) GPTQ matrix with the same scales and qzeros: every
// kernel of the plain path applies, the prefill's dequant-to-LDS included.
#include <algorithm>

#include "device_common.h"
#include "launch.h"

namespace w4a16 {

// qout[jp, n] nibble i = nibble (perm[8 jp + i] % 8) of q[perm[8 jp + i] / 8, n], for the R
// output rows jp0 .. jp0 + R - 1 of column n: all 8 R source words are loaded before any is
// used, so that a thread keeps 8 R loads in flight (one output word per thread kept 8, and a
// pass at K = 4096, N = 6144 took 10.2 us against 8.0 with R = 4, kernel trace).
template <int R>
__device__ __forceinline__ void repack_rows(const uint32_t* __restrict__ q,
                                            const int32_t* __restrict__ perm,
                                            uint32_t* __restrict__ qout, int N, int n, int jp0) {
    if (n >= N) return;
    uint32_t v[R][8];
    int src[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            src[r][i] = perm[8 * (jp0 + r) + i];
            v[r][i] = q[(size_t)(src[r][i] >> 3) * N + n];
        }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= ((v[r][i] >> (4 * (src[r][i] & 7))) & 0xFu) << (4 * i);
        qout[(size_t)(jp0 + r) * N + n] = w;
    }
}

// Grid (ceil(N / 256), K / 8 / R), 256 threads: R output words per thread, columns coalesced.
template <int R>
__global__ void __launch_bounds__(256)
gptq_repack_rows_kernel(const uint32_t* __restrict__ q, const int32_t* __restrict__ perm,
                        uint32_t* __restrict__ qout, int K, int N) {
    repack_rows<R>(q, perm, qout, N, (int)blockIdx.x * 256 + (int)threadIdx.x, (int)blockIdx.y * R);
}

// xout[m, j] = x[m, perm[j]] (perm entries outside [0, K) read column K - 1). Grid
// (ceil(K / 2048), M), 256 threads x 8 columns.
__global__ void __launch_bounds__(256)
gather_columns_kernel(const half_t* __restrict__ x, const int32_t* __restrict__ perm,
                      half_t* __restrict__ xout, int K) {
    const int j0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    const size_t row = (size_t)blockIdx.y * K;
    if (j0 >= K) return;
    if (j0 + 8 <= K) {
        half8_t v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = x[row + min((uint32_t)perm[j0 + i], (uint32_t)K - 1u)];
        *reinterpret_cast<half8_t*>(xout + row + j0) = v;
    } else {
        for (int j = j0; j < K; ++j) xout[row + j] = x[row + min((uint32_t)perm[j], (uint32_t)K - 1u)];
    }
}

// xout[m, j] = x[m, perm[j]] with the row staged in LDS: one workgroup per row, read and
// written with 16-byte coalesced accesses, the permutation applied to the LDS copy (a gather
// straight from global memory costs one cache request per element). Needs K % 8 == 0, K <=
// GATHER_LDS_MAX_K and 16-byte aligned x, perm and xout; entries of perm outside [0, K) read
// column K - 1 instead of memory past the row.
constexpr int GATHER_LDS_MAX_K = 32768;   // 64 KiB of LDS

__device__ __forceinline__ void gather_row_lds(const half_t* __restrict__ x,
                                               const int32_t* __restrict__ perm,
                                               half_t* __restrict__ xout, int K, int per,
                                               int row_i, int part, half_t* row_s) {
    const size_t row = (size_t)row_i * K;
    const int chunks = K / 8;
    const u32x4* src = reinterpret_cast<const u32x4*>(x + row);
    const u32x4* pp = reinterpret_cast<const u32x4*>(perm);
    u32x4* dst = reinterpret_cast<u32x4*>(xout + row);
    const uint32_t last = (uint32_t)K - 1u;
    // this workgroup's share of the row's 8-column output chunks; the perm entries of the
    // thread's first PF chunks are fetched before the row is staged, so that the two latencies
    // overlap
    const int c_beg = part * per + (int)threadIdx.x;
    const int c_end = min(chunks, (part + 1) * per);
    constexpr int PF = 2;
    u32x4 pf[PF][2];
#pragma unroll
    for (int i = 0; i < PF; ++i)
        if (c_beg + 256 * i < c_end) {
            pf[i][0] = pp[2 * (c_beg + 256 * i)];
            pf[i][1] = pp[2 * (c_beg + 256 * i) + 1];
        }
    for (int c = threadIdx.x; c < chunks; c += 256) reinterpret_cast<u32x4*>(row_s)[c] = src[c];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        const int c = c_beg + 256 * i;
        if (c < c_end) {
            const uint32_t idx[8] = {pf[i][0].x, pf[i][0].y, pf[i][0].z, pf[i][0].w,
                                     pf[i][1].x, pf[i][1].y, pf[i][1].z, pf[i][1].w};
            half8_t v;
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = row_s[min(idx[e], last)];
            dst[c] = __builtin_bit_cast(u32x4, v);
        }
    }
    for (int c = c_beg + 256 * PF; c < c_end; c += 256) {
        const u32x4 p0 = pp[2 * c], p1 = pp[2 * c + 1];
        const uint32_t idx[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        half8_t v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = row_s[min(idx[i], last)];
        dst[c] = __builtin_bit_cast(u32x4, v);
    }
}

__global__ void __launch_bounds__(256)
gather_columns_lds_kernel(const half_t* __restrict__ x, const int32_t* __restrict__ perm,
                          half_t* __restrict__ xout, int K, int per) {
    extern __shared__ __attribute__((aligned(16))) half_t row_s[];
    gather_row_lds(x, perm, xout, K, per, (int)blockIdx.x, (int)blockIdx.y, row_s);
}

// The act-order route's two per-call passes in one launch: the gather of x's columns (tasks
// a = row * shares + part, as gather_columns_lds_kernel) and the row repack (tasks r = jq * CX
// + cx, 4 packed rows x 256 columns each, as gptq_repack_rows_kernel<4>). The 1-D grid comes
// in rounds of 8 workgroups, each round all gather or all repack (rounds dealt out in
// proportion): the dispatcher gives workgroup b to XCD b % 8, so repack task r runs on XCD
// r % 8, and with CX % 8 == 0 every column chunk's repack stays on one XCD, whose L2 then
// serves the 8 reads of each source word.
__global__ void __launch_bounds__(256)
act_order_stage_kernel(const uint32_t* __restrict__ q, const int32_t* __restrict__ perm,
                       uint32_t* __restrict__ qout, const half_t* __restrict__ x,
                       half_t* __restrict__ xout, int K, int N, int per, int shares, int g_tasks,
                       int g_rounds, int rounds) {
    extern __shared__ __attribute__((aligned(16))) half_t row_s[];
    const int rho = (int)blockIdx.x >> 3, lam = (int)blockIdx.x & 7;
    const int gb = (int)(((int64_t)rho * g_rounds) / rounds);         // gather rounds before
    const int ga = (int)(((int64_t)(rho + 1) * g_rounds) / rounds);
    if (ga > gb) {   // uniform
        const int a = 8 * gb + lam;
        if (a < g_tasks) gather_row_lds(x, perm, xout, K, per, a / shares, a % shares, row_s);
        return;
    }
    const int cx_n = (N + 255) / 256;
    const int r = 8 * (rho - gb) + lam;
    const int jq = r / cx_n, cx = r - jq * cx_n;
    if (jq < K / 32) repack_rows<4>(q, perm, qout, N, cx * 256 + (int)threadIdx.x, 4 * jq);
}

// Group order on the device, per call: perm[j] = the row of W at position j when the rows are
// sorted by g_idx, stable in k (the order w4a16_prepare_act_order computes on the host), and
// gate[0] = 1 when every group holds exactly G rows (group g then occupies rows [g G, g G + G)
// of that order, as the prefill kernel assumes), else 0 with perm the identity (so that the
// kernels reading it stay in bounds). One workgroup of 16 waves; wave w takes rows
// [w P, w P + P), P = ceil(K / 16) <= 2048, lane l rows w P + l + 64 i (i < 32): it loads all
// of its g_idx entries at once into registers, counts them per group (LDS atomics), the counts
// become each wave's starting position per group (wave order), then the wave places its rows
// 64 at a time, each lane after the earlier lanes of its 64 with the same group (found with one
// ballot per bit of the group index; 64 lane-by-lane compares instead cost 16 us at K = 4096,
// the 16 waves sharing one CU's four SIMDs).
// hdr[0] is the gate word; hdr[1..3] and gcopy (K entries) remember what the last run on these
// buffers computed from (valid flag, K, G, and a copy of g_idx): when all of them match, perm
// and the gate word already hold this call's result and the kernel returns after the compare
// (one load of g_idx and of the copy; a layer's g_idx is the same on every call). The caller
// clears hdr when it allocates the buffers.
// K <= 32768, K / G <= 1024.
constexpr int ORDER_MAX_GROUPS = 1024;
constexpr int ORDER_PER_LANE = 32;   // 32768 rows / 16 waves / 64 lanes

__global__ void __launch_bounds__(1024)
act_order_perm_kernel(const int32_t* __restrict__ g_idx, int32_t* __restrict__ perm,
                      uint32_t* __restrict__ hdr, int32_t* __restrict__ gcopy, int K, int G) {
    __shared__ int pos[16][ORDER_MAX_GROUPS];   // counts, then next position, per (wave, group)
    __shared__ int bad, differ;
    const int groups = K / G;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (K + 15) / 16;
    const int k0 = min(K, w * per), k1 = min(K, k0 + per);
    int gv[ORDER_PER_LANE], cv[ORDER_PER_LANE];
#pragma unroll
    for (int i = 0; i < ORDER_PER_LANE; ++i) {
        const int k = k0 + lane + 64 * i;
        gv[i] = k < k1 ? g_idx[k] : -1;
        cv[i] = k < k1 ? gcopy[k] : -1;
    }
    if (t == 0) {
        bad = 0;
        differ = !(hdr[1] == 1u && hdr[2] == (uint32_t)K && hdr[3] == (uint32_t)G);
    }
    __syncthreads();
    // the order the last call on this buffer computed holds when its g_idx copy, K and G match
    bool mine = false;
#pragma unroll
    for (int i = 0; i < ORDER_PER_LANE; ++i) mine |= gv[i] != cv[i];
    if (mine) differ = 1;
    __syncthreads();
    if (!differ) return;   // uniform: perm and the gate word stay as they are
    for (int i = t; i < 16 * ORDER_MAX_GROUPS; i += 1024) (&pos[0][0])[i] = 0;
#pragma unroll
    for (int i = 0; i < ORDER_PER_LANE; ++i) {
        const int k = k0 + lane + 64 * i;
        if (k < k1) gcopy[k] = gv[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ORDER_PER_LANE; ++i) {
        const int k = k0 + lane + 64 * i;
        if (k < k1) {
            if ((unsigned)gv[i] >= (unsigned)groups) bad = 1;
            else atomicAdd(&pos[w][gv[i]], 1);
        }
    }
    __syncthreads();
    for (int g = t; g < groups; g += 1024) {
        int run = g * G, total = 0;
        for (int v = 0; v < 16; ++v) {
            const int c = pos[v][g];
            pos[v][g] = run;
            run += c;
            total += c;
        }
        if (total != G) bad = 1;
    }
    __syncthreads();
    if (bad) {   // uniform
        for (int k = t; k < K; k += 1024) perm[k] = k;
    } else {
#pragma unroll
        for (int i = 0; i < ORDER_PER_LANE; ++i) {
            if (k0 + 64 * i >= k1) break;   // uniform in the wave
            const int k = k0 + lane + 64 * i;
            const int g = gv[i];            // -1 past the wave's rows
            // lanes holding the same group: one ballot per bit of the group index, each lane
            // keeping the lanes that agree with it on that bit; the rank counts those below it
            uint64_t same = __ballot(g >= 0);
            for (int j = 0; (1 << j) < groups; ++j) {   // uniform
                const uint64_t b = __ballot((g >> j) & 1);
                same &= ((g >> j) & 1) ? b : ~b;
            }
            const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
            const int base = g >= 0 ? pos[w][g] : 0;
            // every lane has read its base (one LDS read of the wave) before any lane adds
            __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
            if (g >= 0) {
                perm[base + rank] = k;
                atomicAdd(&pos[w][g], 1);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
        }
    }
    __syncthreads();
    if (t == 0) {
        hdr[0] = bad ? 0u : 1u;
        hdr[2] = (uint32_t)K;
        hdr[3] = (uint32_t)G;
        hdr[1] = 1u;
    }
}

hipError_t launch_act_order_perm(const int32_t* g_idx, int32_t* perm, uint32_t* hdr, int32_t* gcopy,
                                 int K, int G, hipStream_t st) {
    (void)hipGetLastError();
    if (K < 1 || K > 32768 || G < 1 || K % G || K / G > ORDER_MAX_GROUPS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(act_order_perm_kernel, dim3(1), dim3(1024), 0, st, g_idx, perm, hdr, gcopy, K, G);
    return hipGetLastError();
}

hipError_t launch_gptq_repack_rows(const uint32_t* q, const int32_t* perm, uint32_t* qout, int K,
                                   int N, hipStream_t st) {
    (void)hipGetLastError();
    if (K % 32 == 0)
        hipLaunchKernelGGL(gptq_repack_rows_kernel<4>, dim3((N + 255) / 256, K / 32), dim3(256), 0, st, q,
                           perm, qout, K, N);
    else
        hipLaunchKernelGGL(gptq_repack_rows_kernel<1>, dim3((N + 255) / 256, K / 8), dim3(256), 0, st, q,
                           perm, qout, K, N);
    return hipGetLastError();
}

hipError_t launch_act_order_stage(const uint32_t* q, const int32_t* perm, uint32_t* qout,
                                  const half_t* x, half_t* xout, int M, int K, int N,
                                  hipStream_t st) {
    const int chunks = K / 8;
    const int share = std::max(1, std::min(chunks / 32, 256 / std::max(M, 1)));
    const int per = (chunks + share - 1) / share;
    const int shares = (chunks + per - 1) / per;
    const int64_t g_tasks = (int64_t)M * shares;
    const int64_t r_tasks = (int64_t)((N + 255) / 256) * (K / 32);
    const int64_t g_rounds = (g_tasks + 7) / 8, rounds = g_rounds + (r_tasks + 7) / 8;
    const bool fused = K % 32 == 0 && K <= GATHER_LDS_MAX_K && M >= 1 && rounds * 8 < (1ll << 31) &&
                       reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(perm) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(xout) % 16 == 0;
    if (!fused) {
        hipError_t e = launch_gptq_repack_rows(q, perm, qout, K, N, st);
        return e == hipSuccess ? launch_gather_columns(x, perm, xout, M, K, st) : e;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(act_order_stage_kernel, dim3((unsigned)(rounds * 8)), dim3(256),
                       (size_t)K * sizeof(half_t), st, q, perm, qout, x, xout, K, N, per, shares,
                       (int)g_tasks, (int)g_rounds, (int)rounds);
    return hipGetLastError();
}

hipError_t launch_gather_columns(const half_t* x, const int32_t* perm, half_t* xout, int M, int K,
                                 hipStream_t st) {
    (void)hipGetLastError();
    const bool lds_ok = K % 8 == 0 && K <= GATHER_LDS_MAX_K &&
                        reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(perm) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(xout) % 16 == 0;
    if (lds_ok) {
        constexpr int MAX_BLOCKS = 1 << 30;
        for (int m0 = 0; m0 < M; m0 += MAX_BLOCKS) {
            const int rows = M - m0 < MAX_BLOCKS ? M - m0 : MAX_BLOCKS;
            // a few rows: each row's output chunks are shared by several workgroups (each
            // stages the whole row), so that ~256 workgroups run (M=16, K=4096: 16 -> 256)
            const int chunks = K / 8;
            const int share = std::max(1, std::min(chunks / 32, 256 / rows));
            const int per = (chunks + share - 1) / share;
            hipLaunchKernelGGL(gather_columns_lds_kernel, dim3(rows, (chunks + per - 1) / per),
                               dim3(256), (size_t)K * sizeof(half_t), st, x + (size_t)m0 * K,
                               perm, xout + (size_t)m0 * K, K, per);
        }
        return hipGetLastError();
    }
    constexpr int MAX_ROWS = 32768;   // grid y per launch
    for (int m0 = 0; m0 < M; m0 += MAX_ROWS) {
        const int rows = M - m0 < MAX_ROWS ? M - m0 : MAX_ROWS;
        hipLaunchKernelGGL(gather_columns_kernel, dim3((K + 2047) / 2048, rows), dim3(256), 0, st,
                           x + (size_t)m0 * K, perm, xout + (size_t)m0 * K, K);
    }
    return hipGetLastError();
}

}  // namespace w4a16
