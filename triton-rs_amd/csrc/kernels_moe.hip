// Fused-MoE pieces around the grouped W4A16 GEMM (kernels_prefill.hip, grouped mode).
// The reference has no MoE kernel; the only piece it defines is the activation between the
// expert GEMMs, fused_silu_mul_interleaved_f16 (crates/triton-kernels/src/elementwise.rs:
// 188-212), mirrored here with the same parameters and arithmetic. The rest follows the
// composition the CPU oracle fixes:
//   route:  softmax over the E logits, top-k (ties -> lower expert), weights renormalised
//   align:  (token, slot) pairs sorted by expert, stable in pair index p = t * topk + j,
//           each expert padded to a multiple of block_m with the sentinel P = T * topk
//   gemm1:  h[p]  = f16(x[p / topk] @ W13[e])          (grouped, N = 2 I)
//   act:    a[p]  = f16(silu(f32 h[p][:I]) * f32 h[p][I:])
//   gemm2:  yp[p] = f16(a[p] @ W2[e])                  (grouped, N = K)
//   sum:    y[t]  = f16(sum_j w[t, j] * f32 yp[t * topk + j])
#include "device_common.h"
#include "launch.h"

namespace w4a16 {

// ------------------------------------------------------------------ route

// One thread per token. Top-k is taken on the logits (softmax is monotonic, so the choice
// is the same and is exact); the weight of a chosen expert is its softmax probability, or,
// renormalised over the chosen k, exp(l - l_max) / sum over the chosen of exp(l - l_max).
__global__ void __launch_bounds__(256)
moe_route_kernel(const float* __restrict__ logits, int T, int E, int topk, int renormalize,
                 int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const float* l = logits + (size_t)t * E;
    float mx = l[0];
    for (int e = 1; e < E; ++e) mx = fmaxf(mx, l[e]);
    float denom = 0.f;
    for (int e = 0; e < E; ++e) denom += expf(l[e] - mx);
    uint64_t used[4] = {0, 0, 0, 0};                 // E <= 256
    float sel_sum = 0.f;
    for (int j = 0; j < topk; ++j) {
        int best = -1;
        float bv = 0.f;
        for (int e = 0; e < E; ++e) {
            if ((used[e >> 6] >> (e & 63)) & 1ull) continue;
            if (best < 0 || l[e] > bv) { best = e; bv = l[e]; }   // strict >: lower index wins ties
        }
        used[best >> 6] |= 1ull << (best & 63);
        const float pe = expf(bv - mx);
        ids[(size_t)t * topk + j] = best;
        weights[(size_t)t * topk + j] = pe;
        sel_sum += pe;
    }
    const float inv = 1.0f / (renormalize ? sel_sum : denom);
    for (int j = 0; j < topk; ++j) weights[(size_t)t * topk + j] *= inv;
}

hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int renormalize,
                            int32_t* ids, float* weights, hipStream_t st) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(moe_route_kernel, dim3((T + 255) / 256), dim3(256), 0, st, logits, T, E,
                       topk, renormalize, ids, weights);
    return hipGetLastError();
}

// ------------------------------------------------------------------ align

// One workgroup of 1024 threads. Counts per expert, pads, lays the experts out in order and
// places every pair at start[e] + (number of earlier pairs of the same expert), which keeps
// the order stable. The rank is built per chunk of 1024 pairs from wave ballots and a prefix
// over the 16 waves: up to ALIGN_FAST_E experts every wave takes all its ballots first and
// one table of wave totals serves all experts (3 barriers per chunk); above that, expert by
// expert (3 barriers per expert and chunk).
// With `tiles`, it also lists expert tiles for the grouped GEMM: the cnt[e] rows of expert e
// split into ceil(cnt[e] / tile_bm) tiles of equal height (rounded up to 16 rows, the last
// one shorter), each {first sorted row, rows, e, 0}, experts in order, and their number in
// *num_tiles. A tile never reaches into the padding, so the GEMM computes no padded block.
constexpr int ALIGN_THREADS = 1024;
constexpr int ALIGN_MAX_E = 1024;
constexpr int ALIGN_FAST_E = 64;   // experts ranked with the per-wave ballot table

__global__ void __launch_bounds__(ALIGN_THREADS)
moe_align_kernel(const int32_t* __restrict__ ids, int P, int E, int block_m, int capacity,
                 int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                 int32_t* __restrict__ num_post_padded, int tile_bm, int32_t* __restrict__ tiles,
                 int32_t* __restrict__ num_tiles, uint32_t* __restrict__ counters, int n_counters) {
    __shared__ int cnt[ALIGN_MAX_E];
    __shared__ int start[ALIGN_MAX_E];
    __shared__ int wave_tot[ALIGN_THREADS / 64];
    __shared__ int wtab[ALIGN_FAST_E][ALIGN_THREADS / 64];
    __shared__ int total_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    for (int e = tid; e < E; e += ALIGN_THREADS) cnt[e] = 0;
    // split-K counters of the grouped GEMMs that follow start at zero on every call
    for (int i = tid; i < n_counters; i += ALIGN_THREADS) counters[(size_t)i * FLAG_STRIDE] = 0u;
    __syncthreads();
    // ids outside [0, E) (caller data) are dropped: such a pair is listed in no block
    for (int p = tid; p < P; p += ALIGN_THREADS) {
        const int e = ids[p];
        if ((unsigned)e < (unsigned)E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            start[e] = acc;
            acc += (cnt[e] + block_m - 1) / block_m * block_m;
        }
        total_sh = acc;
        *num_post_padded = acc;
        if (tiles) {
            int n_tiles = 0;
            for (int e = 0; e < E; ++e) {
                const int c = cnt[e];
                const int n = (c + tile_bm - 1) / tile_bm;
                const int per = ((c + n - 1) / max(n, 1) + 15) / 16 * 16;   // <= tile_bm
                for (int r0 = 0; r0 < c; r0 += per, ++n_tiles) {
                    int32_t* td = tiles + 4 * n_tiles;
                    td[0] = start[e] + r0;
                    td[1] = min(per, c - r0);
                    td[2] = e;
                    td[3] = 0;
                }
            }
            *num_tiles = n_tiles;
        }
    }
    __syncthreads();
    const int total = total_sh;
    // sentinel everywhere first, then expert ids per block
    for (int i = tid; i < capacity; i += ALIGN_THREADS) sorted_ids[i] = P;
    for (int e = tid; e < E; e += ALIGN_THREADS) {
        const int b0 = start[e] / block_m;
        const int nb = (cnt[e] + block_m - 1) / block_m;
        for (int b = 0; b < nb; ++b) expert_ids[b0 + b] = e;
        cnt[e] = 0;   // reused below as the running count of placed pairs
    }
    for (int b = total / block_m + tid; b < capacity / block_m; b += ALIGN_THREADS)
        expert_ids[b] = 0;   // blocks past the padded count are never read; keep them valid
    // the sentinel stores must land before any wave overwrites one of them below
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();

    if (E <= ALIGN_FAST_E) {
        // each wave ranks its 64 pairs per expert with one ballot each; one table of wave
        // totals per chunk gives the ranks across waves (3 barriers per chunk, not 3 E)
        for (int c0 = 0; c0 < P; c0 += ALIGN_THREADS) {
            const int p = c0 + tid;
            int mine = p < P ? ids[p] : -1;
            if ((unsigned)mine >= (unsigned)E) mine = -1;
            int inwave = 0;
            for (int e = 0; e < E; ++e) {
                const uint64_t bal = __ballot(mine == e);
                if (lane == 0) wtab[e][wave] = __popcll(bal);
                if (mine == e) inwave = __popcll(bal & ((1ull << lane) - 1ull));
            }
            __syncthreads();
            if (mine >= 0) {
                int before = cnt[mine] + inwave;
                for (int w = 0; w < wave; ++w) before += wtab[mine][w];
                sorted_ids[start[mine] + before] = p;
            }
            __syncthreads();
            if (tid < E) {
                int t = 0;
                for (int w = 0; w < ALIGN_THREADS / 64; ++w) t += wtab[tid][w];
                cnt[tid] += t;
            }
            __syncthreads();
        }
        return;
    }
    for (int c0 = 0; c0 < P; c0 += ALIGN_THREADS) {
        const int p = c0 + tid;
        int mine = p < P ? ids[p] : -1;
        if ((unsigned)mine >= (unsigned)E) mine = -1;
        int rank = 0;
        for (int e = 0; e < E; ++e) {
            const uint64_t bal = __ballot(mine == e);
            if (lane == 0) wave_tot[wave] = __popcll(bal);
            __syncthreads();
            if (mine == e) {
                int before = cnt[e];
                for (int w = 0; w < wave; ++w) before += wave_tot[w];
                before += __popcll(bal & ((1ull << lane) - 1ull));
                rank = before;
            }
            __syncthreads();
            if (tid == 0) {
                int s = 0;
                for (int w = 0; w < ALIGN_THREADS / 64; ++w) s += wave_tot[w];
                cnt[e] += s;
            }
            __syncthreads();
        }
        if (mine >= 0) sorted_ids[start[mine] + rank] = p;
    }
}

hipError_t launch_moe_align(const int32_t* ids, int P, int E, int block_m, int capacity,
                            int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_padded,
                            hipStream_t st, int tile_bm, int32_t* tiles, int32_t* num_tiles,
                            uint32_t* counters, int n_counters) {
    (void)hipGetLastError();
    if (E > ALIGN_MAX_E) return hipErrorInvalidValue;
    if (tiles && (tile_bm < 16 || tile_bm % 16 || !num_tiles)) return hipErrorInvalidValue;
    if (n_counters && !counters) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(ALIGN_THREADS), 0, st, ids, P, E, block_m,
                       capacity, sorted_ids, expert_ids, num_post_padded, tile_bm, tiles,
                       num_tiles, counters, n_counters);
    return hipGetLastError();
}

// ------------------------------------------------------------------ activation

// out[b, i] = f16(silu(g) * u), g = gate_up[b, i], u = gate_up[b, inter + i], silu computed
// in f32 as g / (1 + exp(-g)) (elementwise.rs:188-212). Eight outputs per thread where inter
// and total are multiples of 8 and both buffers 16-byte aligned; one per thread otherwise
// (any inter, and a last row cut short when total is not a multiple of inter, as the
// reference's masked kernel allows).
__global__ void __launch_bounds__(256)
silu_mul_kernel(const half_t* __restrict__ gate_up, half_t* __restrict__ out, int inter,
                int64_t total) {
    const int64_t i8 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i8 >= total) return;
    const int64_t b = i8 / inter, i = i8 - b * inter;
    const half_t* g = gate_up + b * 2 * inter + i;
    const half8_t gv = *reinterpret_cast<const half8_t*>(g);
    const half8_t uv = *reinterpret_cast<const half8_t*>(g + inter);
    half8_t o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = silu_mul_f16(gv[k], uv[k]);
    *reinterpret_cast<half8_t*>(out + i8) = o;
}

// Any inter and any alignment: one output per thread.
__global__ void __launch_bounds__(256)
silu_mul_scalar_kernel(const half_t* __restrict__ gate_up, half_t* __restrict__ out, int inter,
                       int64_t total) {
    const int64_t i1 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i1 >= total) return;
    const int64_t b = i1 / inter, i = i1 - b * inter;
    const half_t* g = gate_up + b * 2 * inter + i;
    out[i1] = silu_mul_f16(g[0], g[inter]);
}

hipError_t launch_silu_mul(const half_t* gate_up, half_t* out, int inter, int64_t total,
                           hipStream_t st) {
    (void)hipGetLastError();
    const bool vec = inter % 8 == 0 && total % 8 == 0 && (reinterpret_cast<uintptr_t>(gate_up) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    if (vec) {
        const int64_t threads = total / 8;
        hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                           st, gate_up, out, inter, total);
    } else {
        hipLaunchKernelGGL(silu_mul_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                           0, st, gate_up, out, inter, total);
    }
    return hipGetLastError();
}

// f32 twin (elementwise.rs:214-250): out[b, i] = silu(g) * u in f32. Four outputs per thread
// where inter and total are multiples of 4 and both buffers 16-byte aligned; one otherwise.
__global__ void __launch_bounds__(256)
silu_mul_f32_kernel(const float* __restrict__ gate_up, float* __restrict__ out, int inter,
                    int64_t total) {
    const int64_t i4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i4 >= total) return;
    const int64_t b = i4 / inter, i = i4 - b * inter;
    const float* g = gate_up + b * 2 * inter + i;
    const float4 gv = *reinterpret_cast<const float4*>(g);
    const float4 uv = *reinterpret_cast<const float4*>(g + inter);
    *reinterpret_cast<float4*>(out + i4) =
        make_float4(silu_mul_f32(gv.x, uv.x), silu_mul_f32(gv.y, uv.y), silu_mul_f32(gv.z, uv.z),
                    silu_mul_f32(gv.w, uv.w));
}

__global__ void __launch_bounds__(256)
silu_mul_f32_scalar_kernel(const float* __restrict__ gate_up, float* __restrict__ out, int inter,
                           int64_t total) {
    const int64_t i1 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i1 >= total) return;
    const int64_t b = i1 / inter, i = i1 - b * inter;
    const float* g = gate_up + b * 2 * inter + i;
    out[i1] = silu_mul_f32(g[0], g[inter]);
}

hipError_t launch_silu_mul_f32(const float* gate_up, float* out, int inter, int64_t total,
                               hipStream_t st) {
    (void)hipGetLastError();
    const bool vec = inter % 4 == 0 && total % 4 == 0 && (reinterpret_cast<uintptr_t>(gate_up) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    if (vec) {
        const int64_t threads = total / 4;
        hipLaunchKernelGGL(silu_mul_f32_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                           st, gate_up, out, inter, total);
    } else {
        hipLaunchKernelGGL(silu_mul_f32_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                           0, st, gate_up, out, inter, total);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ combine

// y[t, n] = f16(sum_j w[t, j] * f32(yp[t * topk + j, n])), eight columns per thread.
__global__ void __launch_bounds__(256)
moe_sum_kernel(const half_t* __restrict__ yp, const float* __restrict__ w, half_t* __restrict__ y,
               int T, int topk, int K) {
    const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (idx >= (int64_t)T * K) return;
    const int t = (int)(idx / K), n = (int)(idx - (int64_t)t * K);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < topk; ++j) {
        const float wj = w[(size_t)t * topk + j];
        const half8_t v = *reinterpret_cast<const half8_t*>(yp + ((size_t)t * topk + j) * K + n);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += wj * (float)v[k];
    }
    half8_t o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = (half_t)acc[k];
    *reinterpret_cast<half8_t*>(y + idx) = o;
}

hipError_t launch_moe_sum(const half_t* y_pairs, const float* weights, half_t* out, int T,
                          int topk, int K, hipStream_t st) {
    (void)hipGetLastError();
    const int64_t threads = (int64_t)T * K / 8;
    hipLaunchKernelGGL(moe_sum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       y_pairs, weights, out, T, topk, K);
    return hipGetLastError();
}

}  // namespace w4a16
