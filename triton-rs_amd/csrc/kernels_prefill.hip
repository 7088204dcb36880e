// Prefill-regime W4A16 GEMM (large M): MFMA-bound, dequant-to-LDS.
//
// C[m, n] = sum_k x[m, k] * W16[k, n], W16 = RNE_f16((q - z) * s) bit-exactly as the
// reference dequantises (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:246-260,
// awq_gemm_int4_typed.rs:213-228); f16 x f16 products accumulated in fp32 with
// v_mfma_f32_16x16x32_f16 (the reference's tt.dot, :265 / :233); fp16 store.
//
// Workgroup tile BM x 256 (BM = 128 or 256), 64 k per stage, 256 threads as 2 x 2 waves,
// each wave (BM/2) x 128. Per stage every thread loads 8 packed words and its 16-byte
// chunks of activations; the words are dequantised once per workgroup into an fp16 B tile
// in LDS ([n][k], k contiguous) and the activations are copied to an A tile ([m][k]).
// Both tiles are double-buffered: the global loads of stage s+1 are issued before the
// MFMAs of stage s, and their dequantisation is interleaved with those MFMAs (one basic
// block, ordered with sched_group_barrier) so VALU work runs while the MFMA pipe is busy.
//
// LDS layout: rows of 64 halfs + 8 halfs of padding (9 units of 16 bytes). A reads (16
// lanes on 16 consecutive rows, same k chunk) are conflict-free with the padding alone.
// B is written column by column by lanes 8 columns apart, so B's 16-byte k chunks are
// XOR-swizzled with (n / 8) % 8; reads (16 consecutive columns) stay conflict-free.
//
// k order inside a chunk of 8: GPTQ words are unpacked as (k0,k4)(k1,k5)(k2,k6)(k3,k7) and
// A is staged in that same order; AWQ keeps natural order (rows paired with v_perm_b32).
#include "device_common.h"
#include "launch.h"

namespace w4a16 {

namespace {
constexpr int BN = 256, BK = 64, LD = BK + 8;   // LDS row: 72 halfs = 9 x 16 bytes

__device__ __forceinline__ half2_t deq2(half2_t h, half2_t hz, half2_t hs) { return (h - hz) * hs; }
__device__ __forceinline__ u32x4 pack8(half2_t a, half2_t b, half2_t c, half2_t d) {
    return u32x4{as_u32(a), as_u32(b), as_u32(c), as_u32(d)};
}
// 16-byte chunk index of k-chunk `kc` (0..7) in B row n
__device__ __forceinline__ int bswz(int n, int kc) { return kc ^ ((n >> 3) & 7); }
}  // namespace

template <int FMT, int BM, int D, bool MOE>
__global__ void __launch_bounds__(256) prefill_kernel(PrefillParams p) {
    constexpr int WM = BM / 2;          // rows per wave
    constexpr int RB = WM / 16;         // row blocks per wave
    constexpr int CB = 8;               // column blocks per wave (128 columns)
    constexpr int ACH = BM * 8 / 256;   // 16-byte A chunks per thread per stage

    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* As = lds;                        // [2][BM][LD]
    half_t* Bs = lds + 2 * BM * LD;          // [2][BN][LD]

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int j = lane & 15, kb = lane >> 4;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int NW = p.N >> 3;
    const int nstages = p.K / BK;

    // Grouped (fused-MoE) mode: row tile blockIdx.y is one BM-row block of expert-sorted
    // (token, slot) pairs; its rows are gathered from the activations through sorted_ids and
    // its results scattered back by pair index; the block's expert selects the weights.
    if constexpr (MOE) {
        if (m0 >= *p.num_post_padded) return;      // uniform: past the padded pair count
        const int e = p.expert_ids[blockIdx.y];
        p.qweight += (size_t)e * p.qweight_stride;
        p.scales += (size_t)e * p.scales_stride;
        if (p.qzeros) p.qzeros += (size_t)e * p.qzeros_stride;
    }
    // source row of tile row `row` (or -1: padding / past M)
    auto src_row = [&](int row) -> int {
        if constexpr (MOE) {
            const int pair = p.sorted_ids[m0 + row];
            return pair < p.num_pairs ? pair / p.a_div : -1;
        } else {
            return m0 + row < p.M ? m0 + row : -1;
        }
    };
    auto dst_row = [&](int row) -> int {
        if constexpr (MOE) {
            const int pair = p.sorted_ids[m0 + row];
            return pair < p.num_pairs ? pair : -1;
        } else {
            return m0 + row < p.M ? m0 + row : -1;
        }
    };
    int arow[ACH];
#pragma unroll
    for (int q = 0; q < ACH; ++q) arow[q] = src_row((t + 256 * q) >> 3);

    // ---- per-thread B assignment: 8 columns (one qzeros word) x 8 k
    //   GPTQ: packed row br = t / 32 of the stage, columns 8 * (t % 32) + 0..7
    //   AWQ:  rows 8 * (t / 32) + 0..7, word column t % 32
    const int bi = t & 31, br = t >> 5;
    const int bn = n0 + 8 * bi;                       // first column of the thread's 8

    // ring of D stages of global loads held in registers (stage s in slot s % D)
    u32x4 areg[D][ACH];
    uint32_t bw[D][8];
    u32x4 sv[D];                                       // 8 scales
    uint32_t zw[D];                                    // zeros word

    auto load_stage = [&](int u, int s) {
        const int k0 = s * BK;
#pragma unroll
        for (int q = 0; q < ACH; ++q) {
            const int idx = t + 256 * q;
            const int row = idx >> 3, cc = idx & 7;
            // rows past M (or padding pairs) are zero (a clamped, branch-free load measured
            // 1.5x slower here)
            const int m = arow[q];
            (void)row;
            areg[u][q] = (m >= 0) ? *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.K + k0 + 8 * cc)
                                  : u32x4{0u, 0u, 0u, 0u};
        }
        int g;
        if constexpr (FMT == FMT_AWQ) {
            const uint32_t off0 = (uint32_t)(k0 + 8 * br) * (uint32_t)NW + (uint32_t)(bn >> 3);
#pragma unroll
            for (int r = 0; r < 8; ++r)
                bw[u][r] = ld_stream(at_bytes(p.qweight, 4u * (off0 + (uint32_t)r * (uint32_t)NW)));
            g = (k0 + 8 * br) / p.G;
        } else {
            const uint32_t off = (uint32_t)((k0 >> 3) + br) * (uint32_t)p.N + (uint32_t)bn;
            const u32x4 v0 = ld_stream4(at_bytes(p.qweight, 4u * off));
            const u32x4 v1 = ld_stream4(at_bytes(p.qweight, 4u * (off + 4)));
            bw[u][0] = v0.x; bw[u][1] = v0.y; bw[u][2] = v0.z; bw[u][3] = v0.w;
            bw[u][4] = v1.x; bw[u][5] = v1.y; bw[u][6] = v1.z; bw[u][7] = v1.w;
            g = (k0 + 8 * br) / p.G;
        }
        sv[u] = *reinterpret_cast<const u32x4*>(p.scales + (size_t)g * p.N + bn);
        zw[u] = (FMT == FMT_GPTQ_SYM) ? 0u : p.qzeros[(size_t)g * NW + (bn >> 3)];
    };

    auto store_stage = [&](int u, int buf) {
        half_t* A = As + buf * BM * LD;
        half_t* B = Bs + buf * BN * LD;
#pragma unroll
        for (int q = 0; q < ACH; ++q) {
            const int idx = t + 256 * q;
            const int row = idx >> 3, cc = idx & 7;
            u32x4 v = areg[u][q];
            if constexpr (FMT != FMT_AWQ)
                v = u32x4{perm(v.z, v.x, 0x05040100u), perm(v.z, v.x, 0x07060302u),
                          perm(v.w, v.y, 0x05040100u), perm(v.w, v.y, 0x07060302u)};
            *reinterpret_cast<u32x4*>(A + row * LD + 8 * cc) = v;
        }
        // zero points (fp16 1024 + z) and scales of the thread's 8 columns
        half2_t hz[8], hs[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            int z;
            if constexpr (FMT == FMT_GPTQ_SYM) z = 8;
            else if constexpr (FMT == FMT_AWQ) z = nib(zw[u], awq_slot(c));
            else z = nib(zw[u], c) + p.zero_offset;
            const half_t zh = (half_t)(1024 + z);
            hz[c] = half2_t{zh, zh};
            const half2_t s2 = as_h2(sv[u][c >> 1]);
            const half_t sc = (c & 1) ? s2.y : s2.x;
            hs[c] = half2_t{sc, sc};
        }
        if constexpr (FMT == FMT_AWQ) {
            half2_t pr[4][8];   // [row pair][column]
#pragma unroll
            for (int rp = 0; rp < 4; ++rp) {
                const uint32_t a = bw[u][2 * rp], b = bw[u][2 * rp + 1];
                const uint32_t p0 = perm(b, a, 0x05040100u);   // slots 0-3 of both rows
                const uint32_t p1 = perm(b, a, 0x07060302u);   // slots 4-7
#pragma unroll
                for (int sl = 0; sl < 8; ++sl) {
                    const uint32_t src = sl < 4 ? p0 : p1;
                    const int col = awq_col_of_slot(sl);
                    pr[rp][col] = deq2(nib_pair(src >> (4 * (sl & 3))), hz[col], hs[col]);
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int n = 8 * bi + c;
                *reinterpret_cast<u32x4*>(B + n * LD + 8 * bswz(n, br)) =
                    pack8(pr[0][c], pr[1][c], pr[2][c], pr[3][c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t w = bw[u][c];
                const int n = 8 * bi + c;
                *reinterpret_cast<u32x4*>(B + n * LD + 8 * bswz(n, br)) =
                    pack8(deq2(nib_pair(w), hz[c], hs[c]), deq2(nib_pair(w >> 4), hz[c], hs[c]),
                          deq2(nib_pair(w >> 8), hz[c], hs[c]), deq2(nib_pair(w >> 12), hz[c], hs[c]));
            }
        }
    };

    float4_t acc[RB][CB];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[r][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    // MFMAs of one stage from LDS buffer `buf`
    auto compute_stage = [&](int buf) {
        const half_t* A = As + buf * BM * LD + (wm * WM) * LD;
        const half_t* B = Bs + buf * BN * LD + (wn * 128) * LD;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int kc = 4 * ks + kb;
            half8_t af[RB], bf[CB];
#pragma unroll
            for (int r = 0; r < RB; ++r)
                af[r] = *reinterpret_cast<const half8_t*>(A + (16 * r + j) * LD + 8 * kc);
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int n = wn * 128 + 16 * c + j;
                bf[c] = *reinterpret_cast<const half8_t*>(B + (16 * c + j) * LD + 8 * bswz(n, kc));
            }
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int c = 0; c < CB; ++c)
                    acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[r], bf[c], acc[r][c], 0, 0, 0);
        }
    };

    // prologue: stages 0 .. D-1 in flight, stage 0 in LDS
#pragma unroll
    for (int u = 0; u < D; ++u)
        if (u < nstages) load_stage(u, u);
    store_stage(0, 0);
    __syncthreads();

    // Steady state, stage s: MFMAs on LDS buffer s % 2, the loads of stage s + D issued
    // into the ring slot stage s vacated, and stage s + 1 dequantised from its slot into the
    // other LDS buffer. These form one basic block (the last stage is peeled) whose schedule
    // interleaves one MFMA with a few VALU / LDS instructions.
    for (int s0 = 0; s0 + 1 < nstages; s0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int s = s0 + u;
            if (s + 1 >= nstages) break;
            if (s + D < nstages) load_stage(u, s + D);
            compute_stage(s & 1);
            store_stage((u + 1) % D, (s + 1) & 1);
#pragma unroll
            for (int i = 0; i < 2 * RB * CB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // 3 VALU
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // 1 LDS read
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // 1 LDS write
            }
            __syncthreads();
        }
    }
    compute_stage((nstages - 1) & 1);

    // ---- epilogue: lane holds D[4 kb + i][j] of each 16 x 16 block
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = dst_row(wm * WM + 16 * r + 4 * kb + i);
            if (m < 0) continue;
            half_t* dst = p.out + (size_t)m * p.N + n0 + wn * 128 + j;
#pragma unroll
            for (int c = 0; c < CB; ++c) dst[16 * c] = (half_t)acc[r][c][i];
        }
}

// ------------------------------------------------------------------ host side

PrefillShape prefill_shape(int fmt, int M, int N, int K, int G, int num_cus) {
    PrefillShape s{};
    if (M < 1 || N % BN || K % BK || G % 8 || K % G) return s;
    const int col_tiles = N / BN;
    // 256-row tiles when they still give every CU a workgroup, else 128
    s.bm = ((M + 255) / 256) * col_tiles >= num_cus ? 256 : 128;
    s.col_tiles = col_tiles;
    s.row_tiles = (M + s.bm - 1) / s.bm;
    s.lds = (size_t)2 * (s.bm + BN) * LD * sizeof(half_t);
    s.ok = true;
    return s;
}

template <int FMT, int BM, bool MOE>
static void launch_t(const PrefillParams& p, dim3 grid, size_t lds, hipStream_t st) {
    // stages of loads in flight: deeper rings do not fit beside the accumulators (they end
    // up in AGPRs and every use pays an AGPR->VGPR copy)
    constexpr int D = 1;
    static bool attr_set = false;   // dynamic LDS above 64 KiB must be allowed once
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<FMT, BM, D, MOE>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr_set = true;
    }
    hipLaunchKernelGGL((prefill_kernel<FMT, BM, D, MOE>), grid, dim3(256), lds, st, p);
}

template <int FMT, bool MOE>
static void launch_fmt(const PrefillParams& p, int bm, dim3 grid, size_t lds, hipStream_t st) {
    if constexpr (MOE) {
        if (bm == 64) launch_t<FMT, 64, true>(p, grid, lds, st);
        else launch_t<FMT, 128, true>(p, grid, lds, st);
    } else {
        if (bm == 256) launch_t<FMT, 256, false>(p, grid, lds, st);
        else launch_t<FMT, 128, false>(p, grid, lds, st);
    }
}

template <bool MOE>
static hipError_t launch_any(int fmt, const PrefillParams& p, int bm, dim3 grid, size_t lds,
                             hipStream_t st) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (fmt == FMT_AWQ) launch_fmt<FMT_AWQ, MOE>(p, bm, grid, lds, st);
    else if (fmt == FMT_GPTQ) launch_fmt<FMT_GPTQ, MOE>(p, bm, grid, lds, st);
    else launch_fmt<FMT_GPTQ_SYM, MOE>(p, bm, grid, lds, st);
    return hipGetLastError();
}

hipError_t launch_prefill(int fmt, const PrefillParams& p, const PrefillShape& s, hipStream_t st) {
    return launch_any<false>(fmt, p, s.bm, dim3(s.col_tiles, s.row_tiles), s.lds, st);
}

bool moe_gemm_supported(int N, int K, int G, int block_m) {
    return N % BN == 0 && K % BK == 0 && G % 8 == 0 && K % G == 0 &&
           (block_m == 64 || block_m == 128);
}

hipError_t launch_moe_gemm(int fmt, const PrefillParams& p, int block_m, int max_blocks,
                           hipStream_t st) {
    const size_t lds = (size_t)2 * (block_m + BN) * LD * sizeof(half_t);
    return launch_any<true>(fmt, p, block_m, dim3(p.N / BN, max_blocks), lds, st);
}

}  // namespace w4a16
