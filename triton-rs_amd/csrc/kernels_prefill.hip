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
#include <type_traits>

#include "device_common.h"
#include "launch.h"
#include "splitk.h"
#include "lds_dma.h"

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
    if (p.gate && *p.gate != p.gate_want) return;   // uniform: the whole grid returns
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
        if ((unsigned)e >= (unsigned)p.num_experts) return;   // caller data out of range
        p.qweight += (size_t)e * p.qweight_stride;
        p.scales += (size_t)e * p.scales_stride;
        if (p.qzeros) p.qzeros += (size_t)e * p.qzeros_stride;
    }
    // source row of tile row `row` (or -1: padding / past M)
    auto src_row = [&](int row) -> int {
        if constexpr (MOE) {
            const int pair = p.sorted_ids[m0 + row];
            return (unsigned)pair < (unsigned)p.num_pairs ? pair / p.a_div : -1;
        } else {
            return m0 + row < p.M ? m0 + row : -1;
        }
    };
    auto dst_row = [&](int row) -> int {
        if constexpr (MOE) {
            const int pair = p.sorted_ids[m0 + row];
            return (unsigned)pair < (unsigned)p.num_pairs ? pair : -1;
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

// ------------------------------------------------------------------ pipelined variant
//
// Same tile work as prefill_kernel with the memory latency taken off the MFMA stream and two
// waves per SIMD. All global traffic goes straight to LDS with buffer_load ... lds (no
// registers held across stages):
//  * A (activations) into two LDS slots, one stage ahead. Rows past M (or padding pairs)
//    get an offset past the buffer's end, which the buffer unit returns as zero.
//  * the packed words, scales and zeros of B into a three-slot LDS ring, three stages
//    ahead; each stage dequantises the next stage's B from that ring into one of two fp16
//    B tiles.
// Per stage the loads are issued A first, B second, and the stage ends waiting with a vmcnt
// that leaves only the B loads just issued in flight: A(s+1) and everything older is in LDS
// at the barrier, B gets two stages of latency. One stage is 64 k. 8 waves (4 along M, 2
// along N): with one wave per SIMD the dequantisation VALU and the MFMAs do not overlap.
//
// LDS layouts (measured conflict-free for the operand reads and the dequant writes):
//  A [BM][8 chunks of 8 k]: chunk kc of row r at slot kc ^ (r & 7);
//  B [8 chunks][256 columns] of 8 k each: column n at position n ^ ((n >> 3) & 7).
// A is staged in natural k order (GPTQ's unpack order is undone on the B side with
// v_perm_b32).
//
// Variants of the same kernel: dense (rows m0 + r of x); grouped MoE (rows gathered
// through sorted pair ids), over block_m blocks or over expert tiles from a list; and split
// K (grid z = K splits, fp32 partials, the last split of a tile sums them in split order).
namespace {
__device__ __forceinline__ int bpos(int n) { return n ^ ((n >> 3) & 7); }

// One raw ring slot: packed words of a stage (64 k x 256 columns, 8 KB), then 1 KB for the
// group's scales (256 halfs) and 1 KB for its zeros (32 words). Every LDS load instruction
// writes all 64 lanes (lanes out of range write zeros), so each gets a 1 KB region of its own.
constexpr int RAW_W = 8 * 1024;
constexpr int RAW_S = 1024;
constexpr int RAW_ST = RAW_W + 2 * 1024;
}  // namespace

// The B tiles are always 256 columns wide: with BN = 224 the lanes past the tile dequantise
// into columns nobody reads instead of branching around the work.
size_t prefill_dma_lds(int bm, int bn) {
    (void)bn;
    return (size_t)2 * bm * BK * 2 + (size_t)2 * BN * BK * 2 + (size_t)3 * RAW_ST;
}

constexpr int PF_THREADS = 512;   // 8 waves: 4 along M x 2 along N

// XCD-grouped order of an expert-tile grid. The dispatcher hands workgroup b of a launch to
// XCD b mod 8, so a grid in the natural order (column tiles fastest) spreads every expert's
// tile over all eight XCDs, and each XCD's L2 then fetches every expert's activation rows
// (the down projection moved twice its bytes that way). Here the 1-D grid of
// gx * round_up(max_tiles, 8) * gz workgroups is dealt out in units of one expert tile's
// columns, or of 1/c of them: with nt tiles, c = 8 / gcd(nt, 8), so the nt * c units fill
// the eight XCDs evenly, unit u going to XCD u mod 8 and each XCD taking its units one
// after another, all column tiles and K splits of a unit together. A unit's activation rows
// are then fetched into one L2 and reused there by its column tiles. Placement only: the
// results do not depend on it. Returns false for a workgroup with no unit (it exits).
__device__ __forceinline__ bool xcd_tile_of_block(int gx, int gz, int max_tiles, int nt,
                                                  int& bx, int& by, int& bz) {
    const int L = blockIdx.x;
    const int gyp = (max_tiles + 7) & ~7;
    nt = min(nt, max_tiles);
    if (nt <= 0) return false;
    const int low = nt & -nt;
    const int c = 8 / (low < 8 ? low : 8);
    if (gx % c) {   // units would split a column tile: the natural order over the 1-D grid
        bx = L % gx;
        by = (L / gx) % gyp;
        bz = L / (gx * gyp);
        return by < nt;
    }
    const int cw = gx / c, W = cw * gz;   // column tiles per unit, workgroups per unit
    const int slot = L >> 3, i = slot / W;
    if (i >= nt * c / 8) return false;
    const int u = (L & 7) + 8 * i;
    by = u / c;
    const int w = slot - i * W;
    bz = w / cw;
    bx = (u - by * c) * cw + (w - bz * cw);
    return true;
}

// E: the element type of x, the scales and the output. With bf16 (dense checkpoint layouts)
// a weight is RNE_bf16((q - z) * s) (deq2_bf16) and the MFMA is the bf16 one.
template <int FMT, int BM, int BN, bool MOE, typename E = half_t>
__global__ void __launch_bounds__(PF_THREADS) prefill_dma_kernel(PrefillParams p) {
    constexpr bool BF = std::is_same<E, bf16_t>::value;
    typedef typename vec8<E>::type v8_t;
    static_assert(!BF || (!MOE && FMT != FMT_PREP), "bf16: dense checkpoint layouts");
    if (p.gate && *p.gate != p.gate_want) return;   // uniform: the whole grid returns
    constexpr int WGM = 4, WGN = 2, NWV = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;     // wave tile
    constexpr int RB = WM / 16, CB = WN / 16;
    constexpr int A_ST = BM * BK, B_ST = 256 * BK;  // halfs per stage (B: 256 columns)
    constexpr int ADMA = BM * 8 / PF_THREADS;       // A chunks per thread per stage
    constexpr int BWC = BN / 8;                     // 8-column groups of the tile
    static_assert(BWC <= 32 && WN % 16 == 0 && WM % 16 == 0 && ADMA >= 1, "tile shape");

    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* As = lds;                                          // [2][BM][64]
    half_t* Bs = lds + 2 * A_ST;                               // [2][8][256][8]
    char* Raw = reinterpret_cast<char*>(lds + 2 * A_ST + 2 * B_ST);   // [3][RAW_ST]

    const int t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int j = lane & 15, kb = lane >> 4;
    const int ksp = max(p.ksplit, 1);
    // (column tile, row tile, K split) of this workgroup: the grid's own coordinates, or in
    // the XCD-grouped expert-tile order a 1-D grid dealt out by xcd_tile_of_block
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    if constexpr (MOE) {
        if (p.tiles && p.xcd_tiles > 0 &&
            !xcd_tile_of_block(p.N / BN, ksp, p.xcd_tiles, *p.num_tiles, bx, by, bz))
            return;
    }
    int m0 = by * BM, rows = BM;
    (void)rows;
    const int n0 = bx * BN;
    const int NW = p.N >> 3;
    // split K: this workgroup's K stages are [s0, s0 + ns)
    const int ns = p.K / BK / ksp;
    const int s0 = bz * ns;

    if constexpr (MOE) {
        int e;
        if (p.tiles) {   // expert tile: rows past its height are masked like padding
            if (by >= *p.num_tiles) return;
            const int32_t* td = p.tiles + 4 * by;
            m0 = td[0];
            rows = td[1];
            e = td[2];
        } else {
            if (m0 >= *p.num_post_padded) return;
            e = p.expert_ids[by];
            if ((unsigned)e >= (unsigned)p.num_experts) return;   // caller data out of range
        }
        p.qweight += (size_t)e * p.qweight_stride;
        p.scales += (size_t)e * p.scales_stride;
        if (p.qzeros) p.qzeros += (size_t)e * p.qzeros_stride;
    }
    auto src_row = [&](int row) -> int {
        if constexpr (MOE) {
            if (row >= rows) return -1;
            const int pair = p.sorted_ids[m0 + row];
            return (unsigned)pair < (unsigned)p.num_pairs ? pair / p.a_div : -1;
        } else {
            return m0 + row < p.M ? m0 + row : -1;
        }
    };
    auto dst_row = [&](int row) -> int {
        if constexpr (MOE) {
            if (row >= rows) return -1;
            const int pair = p.sorted_ids[m0 + row];
            return (unsigned)pair < (unsigned)p.num_pairs ? pair : -1;
        } else {
            return m0 + row < p.M ? m0 + row : -1;
        }
    };

    // ---- A: chunk (q, wave, lane) of a stage is LDS row idx / 8, slot idx % 8
    const int a_rows = MOE ? (p.num_pairs + p.a_div - 1) / p.a_div : p.M;
    const i32x4_t ars = buffer_rsrc(p.x, (uint32_t)a_rows * (uint32_t)p.K * 2u);
    uint32_t aoff[ADMA];
#pragma unroll
    for (int q = 0; q < ADMA; ++q) {
        const int idx = (q * NWV + wave) * 64 + lane;
        const int row = idx >> 3, slot = idx & 7;
        const int m = src_row(row);
        aoff[q] = m >= 0 ? ((uint32_t)m * (uint32_t)p.K + 8u * (uint32_t)(slot ^ (row & 7))) * 2u
                         : DMA_OOB;
    }
    auto dma_a = [&](int slot, int s) {
        half_t* dst = As + slot * A_ST;
#pragma unroll
        for (int q = 0; q < ADMA; ++q)
            dma16(ars, dst + (q * NWV + wave) * 64 * 8, aoff[q] + (uint32_t)(s0 + s) * (BK * 2));
    };

    // ---- B raw: words of a stage as [64 rows][32 words] (AWQ) or [8 packed rows][256
    // words] (GPTQ) in eight 1 KB blocks, one per wave; scales by wave 0, zeros by the other
    // waves (identical bytes to one place: a harmless race that keeps the stage free of
    // branches)
    // prepared layout: strips of 16 columns, sb bytes each, the table's tb bytes first
    const uint32_t sb = FMT == FMT_PREP ? (uint32_t)prep_strip_bytes(p.K, p.G) : 0u;
    const uint32_t tb = FMT == FMT_PREP ? prep_table_words(p.K, p.G) * 4u : 0u;
    const i32x4_t wrs = buffer_rsrc(p.qweight, FMT == FMT_PREP ? (uint32_t)(p.N / 16) * sb
                                                               : (uint32_t)((size_t)p.K * p.N / 2));
    const i32x4_t srs = buffer_rsrc(p.scales, (uint32_t)((size_t)(p.K / p.G) * p.N * 2));
    const i32x4_t zrs = buffer_rsrc(p.qzeros ? (const void*)p.qzeros : (const void*)p.scales,
                                    p.qzeros ? (uint32_t)((size_t)(p.K / p.G) * NW * 4) : 0u);
    uint32_t woff;
    if constexpr (FMT == FMT_PREP) {
        // a stage is half a block (64 rows, 512 bytes) of each of the tile's 16 strips: wave w
        // loads strips 2 w and 2 w + 1
        const int sl = 2 * wave + (lane >> 5);
        woff = 16 * sl < BN ? (uint32_t)(n0 / 16 + sl) * sb + tb + (uint32_t)(lane & 31) * 16u : DMA_OOB;
    } else if constexpr (FMT == FMT_AWQ) {
        const int row = wave * 8 + (lane >> 3), chunk = lane & 7;   // 4 words per lane
        woff = 4 * chunk < BWC
                   ? ((uint32_t)row * (uint32_t)NW + (uint32_t)(n0 >> 3) + 4u * chunk) * 4u
                   : DMA_OOB;
    } else {
        woff = 4 * lane < BN ? ((uint32_t)wave * (uint32_t)p.N + (uint32_t)n0 + 4u * lane) * 4u
                             : DMA_OOB;                          // packed row `wave`
    }
    const bool zw_wave = FMT != FMT_GPTQ_SYM && FMT != FMT_PREP && wave != 0;
    const i32x4_t szrs = FMT == FMT_PREP ? wrs : zw_wave ? zrs : srs;
    // prepared: the stage's table row (64 bytes of each strip, 1 KB), by wave 0
    const uint32_t szoff = FMT == FMT_PREP ? (16 * (lane >> 2) < BN ? (uint32_t)(n0 / 16 + (lane >> 2)) * sb + (uint32_t)(lane & 3) * 16u : DMA_OOB)
                         : zw_wave ? (lane * 4 < BWC ? ((uint32_t)(n0 >> 3) + 4u * lane) * 4u : DMA_OOB)
                                   : (lane < BWC ? ((uint32_t)n0 + 8u * lane) * 2u : DMA_OOB);
    const uint32_t szrow = zw_wave ? (uint32_t)NW * 4u : (uint32_t)p.N * 2u;   // bytes per group
    const int szdst = RAW_W + (zw_wave ? RAW_S : 0);
    auto dma_b = [&](int slot, int s) {
        char* dst = Raw + slot * RAW_ST;
        const int k0 = (s0 + s) * BK, g = k0 / p.G;
        if constexpr (FMT == FMT_PREP) {
            const int row = (k0 >> 7) * prep_table_rows(p.G) + (p.G < 128 ? (k0 & 127) / p.G : 0);
            if (wave == 0) dma16(szrs, dst + szdst, szoff + (uint32_t)row * 64u);
            dma16(wrs, dst + wave * 1024, woff + (uint32_t)(k0 >> 7) * 1024u + (uint32_t)((k0 >> 6) & 1) * 512u);
            return;
        }
        const uint32_t wstep = (FMT == FMT_AWQ) ? (uint32_t)k0 * (uint32_t)NW * 4u
                                                : (uint32_t)(k0 >> 3) * (uint32_t)p.N * 4u;
        dma16(szrs, dst + szdst, szoff + (uint32_t)g * szrow);
        dma16(wrs, dst + wave * 1024, woff + wstep);
    };

    // ---- dequantisation into the fp16 B tile: thread t owns k chunk kq = t / 64 (8 k) and
    // DQC columns of one 8-column word group bw: columns 8 bw + DQC hh + 0..DQC-1. A tile of
    // 256 (or 224) columns gives each thread 4 columns (bw = t % 32, hh = (t / 32) % 2); a
    // 128-column tile 2 (bw = t % 16, hh = (t / 16) % 4), so no thread dequantises columns
    // outside the tile.
    constexpr int DQC = BN <= 128 ? 2 : 4;
    constexpr int DQW = 8 / DQC;   // column groups per word
    const int bw = DQC == 4 ? (t & 31) : (t & 15);
    const int hh = DQC == 4 ? ((t >> 5) & 1) : ((t >> 4) & 3);
    const int kq = t >> 6;
    // prepared layout: thread t dequantises column pn, half ph (rows 32 ph .. 32 ph + 31 of
    // the stage), words DQC pq .. of its lane chunk
    const int pn = DQC == 4 ? (t & 255) : (t & 127);
    const int ph = DQC == 4 ? (t >> 8) : ((t >> 7) & 1);
    const int pq = DQC == 4 ? 0 : (t >> 8);
    (void)pn; (void)ph; (void)pq;
    static_assert(BN <= 128 || BN >= 192, "tile width");
    (void)DQW;

    // The dequantisation comes in three parts, so that its VALU work can be placed between
    // the MFMAs of a stage: raw reads from the ring slot, per-column arithmetic, LDS writes.
    struct DqRaw { uint32_t sv[2]; uint32_t zw; uint32_t w[8]; uint32_t e[4]; };
    auto dq_load = [&](int slot) {
        DqRaw d;
        const char* src = Raw + slot * RAW_ST;
        if constexpr (FMT == FMT_PREP) {
            // thread (column pn, half ph, part pq): words DQC pq .. DQC pq + DQC - 1 of lane
            // pn % 16 + 16 ph of strip pn / 16 (16-byte lane chunks read whole, conflict-free),
            // and the column's table entry
            const uint32_t* wp = reinterpret_cast<const uint32_t*>(src + (pn >> 4) * 512 + ((pn & 15) + 16 * ph) * 16) + DQC * pq;
            if constexpr (DQC == 4) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(wp);
                d.w[0] = v.x; d.w[1] = v.y; d.w[2] = v.z; d.w[3] = v.w;
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2*>(wp);
                d.w[0] = v.x; d.w[1] = v.y;
            }
            d.e[0] = reinterpret_cast<const uint32_t*>(src + RAW_W)[pn];
            return d;
        }
        const uint32_t* sc32 = reinterpret_cast<const uint32_t*>(src + RAW_W);
        if constexpr (DQC == 4) { d.sv[0] = sc32[4 * bw + 2 * hh]; d.sv[1] = sc32[4 * bw + 2 * hh + 1]; }
        else { d.sv[0] = sc32[4 * bw + hh]; d.sv[1] = 0u; }
        d.zw = 0u;
        if constexpr (FMT != FMT_GPTQ_SYM) d.zw = reinterpret_cast<const uint32_t*>(src + RAW_W + RAW_S)[bw];
        if constexpr (FMT == FMT_AWQ) {
            // rows 8 kq .. 8 kq + 7 of word column bw
            const uint32_t* wp = reinterpret_cast<const uint32_t*>(src) + 8 * kq * 32 + bw;
#pragma unroll
            for (int r = 0; r < 8; ++r) d.w[r] = wp[32 * r];
        } else if constexpr (DQC == 4) {
            // packed row kq (8 k) of columns 8 bw + 4 hh + 0..3
            const u32x4 w4 = *reinterpret_cast<const u32x4*>(src + kq * 1024 + 4 * (8 * bw + 4 * hh));
            d.w[0] = w4.x; d.w[1] = w4.y; d.w[2] = w4.z; d.w[3] = w4.w;
        } else {
            const u32x2 w2 = *reinterpret_cast<const u32x2*>(src + kq * 1024 + 4 * (8 * bw + 2 * hh));
            d.w[0] = w2.x; d.w[1] = w2.y;
        }
        return d;
    };
    // column c (0 .. DQC-1) of the thread's columns, as the 8 k of one B-operand chunk
    auto dq_col = [&](const DqRaw& d, int c) -> u32x4 {
        const int cc = DQC * hh + c;   // column within its 8-column group
        if constexpr (FMT == FMT_PREP) {
            // word c: 8 rows of the thread's column; scale and zero point from the entry;
            // rows in natural order, pairs (2 i, 2 i + 1)
            const uint32_t e = d.e[0], zb = 0x6400u + (e >> 16);
            const half2_t hz = as_h2(zb | (zb << 16)), hs = as_h2(perm(e, e, 0x01000100u));
            const uint32_t w = d.w[c];
            return pack8(deq2(nib_pair(w), hz, hs), deq2(nib_pair(w >> 4), hz, hs),
                         deq2(nib_pair(w >> 8), hz, hs), deq2(nib_pair(w >> 12), hz, hs));
        }
        const uint32_t sw = DQC == 4 ? d.sv[c >> 1] : d.sv[0];
        if constexpr (BF) {
            // the same words and pairs as below, each pair RNE_bf16((q - z) * s)
            const float sf = bf16_bits_to_f32((c & 1) ? sw >> 16 : sw & 0xFFFFu);
            if constexpr (FMT == FMT_AWQ) {
                const int slot = awq_slot(cc);
                const float nzs = -(float)nib(d.zw, slot) * sf;
                uint32_t pr[4];
#pragma unroll
                for (int rp = 0; rp < 4; ++rp) {
                    const uint32_t a = d.w[2 * rp], b = d.w[2 * rp + 1];
                    const uint32_t pp = perm(b, a, (slot & 4) ? 0x07060302u : 0x05040100u);
                    pr[rp] = deq2_bf16(pp >> (4 * (slot & 3)), sf, nzs);
                }
                return u32x4{pr[0], pr[1], pr[2], pr[3]};
            } else {
                const int z = FMT == FMT_GPTQ_SYM ? 8 : nib(d.zw, cc) + p.zero_offset;
                const float nzs = -(float)z * sf;
                const uint32_t w = d.w[c];
                const uint32_t q0 = deq2_bf16(w, sf, nzs), q1 = deq2_bf16(w >> 4, sf, nzs);
                const uint32_t q2 = deq2_bf16(w >> 8, sf, nzs), q3 = deq2_bf16(w >> 12, sf, nzs);
                return u32x4{perm(q1, q0, 0x05040100u), perm(q3, q2, 0x05040100u),
                             perm(q1, q0, 0x07060302u), perm(q3, q2, 0x07060302u)};
            }
        }
        const half2_t hs = as_h2(perm(sw, sw, (c & 1) ? 0x07060706u : 0x05040504u));
        if constexpr (FMT == FMT_AWQ) {
            const int slot = awq_slot(cc);
            const uint32_t zb = 0x6400u + (uint32_t)nib(d.zw, slot);
            const half2_t hz = as_h2(zb | (zb << 16));
            half2_t pr[4];
#pragma unroll
            for (int rp = 0; rp < 4; ++rp) {
                // slots 0-3 (or 4-7) of rows 2 rp and 2 rp + 1 in the low and high halves
                const uint32_t a = d.w[2 * rp], b = d.w[2 * rp + 1];
                const uint32_t pp = perm(b, a, (slot & 4) ? 0x07060302u : 0x05040100u);
                pr[rp] = deq2(nib_pair(pp >> (4 * (slot & 3))), hz, hs);
            }
            return pack8(pr[0], pr[1], pr[2], pr[3]);
        } else {
            uint32_t z;
            if constexpr (FMT == FMT_GPTQ_SYM) z = 8u;
            else z = (uint32_t)(nib(d.zw, cc) + p.zero_offset);
            const uint32_t zb = 0x6400u + z;
            const half2_t hz = as_h2(zb | (zb << 16));
            const uint32_t w = d.w[c];
            const uint32_t q0 = as_u32(deq2(nib_pair(w), hz, hs));         // k0, k4
            const uint32_t q1 = as_u32(deq2(nib_pair(w >> 4), hz, hs));    // k1, k5
            const uint32_t q2 = as_u32(deq2(nib_pair(w >> 8), hz, hs));    // k2, k6
            const uint32_t q3 = as_u32(deq2(nib_pair(w >> 12), hz, hs));   // k3, k7
            return u32x4{perm(q1, q0, 0x05040100u), perm(q3, q2, 0x05040100u),
                         perm(q1, q0, 0x07060302u), perm(q3, q2, 0x07060302u)};
        }
    };
    auto dq_store = [&](int buf, const u32x4 (&col)[DQC]) {
        if constexpr (FMT == FMT_PREP) {   // k chunks 4 ph + DQC pq + c of column pn
#pragma unroll
            for (int c = 0; c < DQC; ++c)
                *reinterpret_cast<u32x4*>(Bs + buf * B_ST + (4 * ph + DQC * pq + c) * 256 * 8 + 8 * bpos(pn)) = col[c];
            return;
        }
        half_t* B = Bs + buf * B_ST + kq * 256 * 8;
#pragma unroll
        for (int c = 0; c < DQC; ++c)
            *reinterpret_cast<u32x4*>(B + 8 * bpos(8 * bw + DQC * hh + c)) = col[c];
    };
    auto dequant_b = [&](int slot, int buf) {
        const DqRaw d = dq_load(slot);
        u32x4 col[DQC];
#pragma unroll
        for (int c = 0; c < DQC; ++c) col[c] = dq_col(d, c);
        dq_store(buf, col);
    };

    float4_t acc[RB][CB];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[r][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Rows of the wave's row blocks: block r covers rows row0 + RSTEP r .. +15. A dense tile
    // gives each wave WM contiguous rows; an expert tile interleaves the blocks over the four
    // wave rows (r WGM + wm), so that a tile filled only partly still spreads its real rows,
    // and the MFMAs they need, evenly over the SIMDs.
    constexpr int RSTEP = MOE ? 16 * WGM : 16;
    const int row0 = MOE ? 16 * wm : wm * WM;

    // operand offsets (halfs) within a stage: A row block r at +RSTEP r rows; B column block c
    int boff[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) boff[c] = (kb * 256 + bpos(wn * WN + 16 * c + j)) * 8;
    const int aoff_l = (row0 + j) * BK;

    // One stage with the MFMAs of the first RV row blocks only (an expert tile's blocks past
    // its rows hold no tokens and are skipped; RV is uniform over the wave).
    auto fused = [&](auto rv, int a_slot, int buf, int raw_slot, int dq_buf) {
        constexpr int RV = decltype(rv)::value;
        const DqRaw d = dq_load(raw_slot);
        const half_t* A = As + a_slot * A_ST + aoff_l;
        const half_t* B = Bs + buf * B_ST;
        u32x4 col[DQC];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int kc = 4 * ks + kb;
            v8_t af[RV > 0 ? RV : 1], bf[CB];
#pragma unroll
            for (int r = 0; r < RV; ++r)
                af[r] = *reinterpret_cast<const v8_t*>(A + RSTEP * r * BK + 8 * (kc ^ (j & 7)));
#pragma unroll
            for (int c = 0; c < CB; ++c)
                if (RV > 0) bf[c] = *reinterpret_cast<const v8_t*>(B + boff[c] + ks * 4 * 256 * 8);
            // checkpoint formats, tiles 224 or 256 wide: the wave's MFMA burst at raised
            // priority, so that the SIMD's other wave, dequantising or reading LDS, does not
            // hold up its issue (same-box A/B: config 3 4096->14336 / 14336->4096 228-231 ->
            // 221-222 us, the MoE layer 0.571 -> 0.559 ms; 256 x 128 tiles, with a third of
            // the MFMAs per burst, 1.5-3 % slower; with the prepared B stage 1-5 % slower)
            constexpr bool PRIO = FMT != FMT_PREP && BN >= 224;
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int r = 0; r < RV; ++r)
#pragma unroll
                for (int c = 0; c < CB; ++c) acc[r][c] = mfma16x16x32(af[r], bf[c], acc[r][c]);
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int c = ks * DQC / 2; c < (ks + 1) * DQC / 2; ++c) col[c] = dq_col(d, c);
            // place the dequantisation arithmetic between the MFMAs: 1 MFMA, 2 VALU
            // (measured 229 -> 216 us at M=2048, K=4096, N=14336 against MFMAs then
            // dequantisation; 1 or 3 VALU per MFMA were slower)
#pragma unroll
            for (int i = 0; i < RV * CB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0); // 2 VALU
            }
        }
        dq_store(dq_buf, col);
    };

    // ---- prologue: raw B of stages 0, 1, 2 and A(0) in flight; dequantise B(0)
    dma_b(0, 0);
    dma_b(1, min(1, ns - 1));
    dma_b(2, min(2, ns - 1));
    dma_a(0, 0);
    wait_vmcnt<0>();
    __syncthreads();
    dequant_b(0, 0);
    __syncthreads();

    // ---- stage s: issue A(s+1), then raw B(s+3) into the ring slot B(s) vacated; MFMAs
    // of stage s with the dequantisation of B(s+1) interleaved; wait for all but the raw
    // word load just issued; barrier. Indices past the end are clamped (their loads land in slots nobody
    // reads any more).
    auto main_loop = [&](auto rv) {
        for (int s = 0; s < ns; ++s) {
            const int rs = s % 3;
            dma_a((s + 1) & 1, min(s + 1, ns - 1));
            dma_b(rs, min(s + 3, ns - 1));
            fused(rv, s & 1, s & 1, rs == 2 ? 0 : rs + 1, (s + 1) & 1);
            wait_vmcnt<1>();
            __syncthreads();
        }
    };
    if constexpr (MOE) {
        // row blocks of this wave that start inside the tile's rows; every variant runs the
        // same stages and barriers
        const int rv = rows <= row0 ? 0 : min(RB, (rows - row0 + RSTEP - 1) / RSTEP);
        if (rv >= RB) main_loop(std::integral_constant<int, RB>{});
        else if (RB > 1 && rv == RB - 1) main_loop(std::integral_constant<int, (RB > 1 ? RB - 1 : RB)>{});
        else if (RB > 2 && rv == RB - 2) main_loop(std::integral_constant<int, (RB > 2 ? RB - 2 : RB)>{});
        else if (RB > 3 && rv == RB - 3) main_loop(std::integral_constant<int, (RB > 3 ? RB - 3 : RB)>{});
        else main_loop(std::integral_constant<int, 0>{});
    } else {
        main_loop(std::integral_constant<int, RB>{});
    }
    wait_vmcnt<0>();   // no LDS write may be in flight when the workgroup ends

    // ---- epilogue: lane holds D[4 kb + i][j] of each 16 x 16 block
    if (ksp > 1) {
        // partials of this split (rows of the output: M rows, or pairs in MoE mode), then
        // the last split of the tile sums all of them in split order (deterministic) and
        // writes the fp16 tile
        __shared__ int last_flag;
        const size_t MN = (size_t)(MOE ? p.num_pairs : p.M) * p.N;
        float* mine = p.ws + (size_t)bz * MN;
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = dst_row(row0 + RSTEP * r + 4 * kb + i);
                if (m < 0) continue;
                float* dst = mine + (size_t)m * p.N + n0 + wn * WN + j;
#pragma unroll
                for (int c = 0; c < CB; ++c) st_partial<SCOPE_DEVICE>(dst + 16 * c, acc[r][c][i]);
            }
        const int tile = by * (p.N / BN) + bx;
        if (!splitk_arrive(splitk_counter(p.counters, tile), ksp, &last_flag)) return;
        constexpr int C4 = BN / 4;
        const int nrows = MOE ? rows : min(BM, p.M - m0);
        for (int idx = t; idx < nrows * C4; idx += PF_THREADS) {
            const int lr = idx / C4, c = 4 * (idx - lr * C4);
            const int m = dst_row(lr);
            if (m < 0) continue;
            const size_t off = (size_t)m * p.N + n0 + c;
            float4_t v = ld_partial4<SCOPE_DEVICE>(p.ws + off);
            for (int sp = 1; sp < ksp; ++sp) v += ld_partial4<SCOPE_DEVICE>(p.ws + sp * MN + off);
            *reinterpret_cast<u32x2*>(p.out + off) = u32x2{pack2(E{}, v.x, v.y), pack2(E{}, v.z, v.w)};
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = dst_row(row0 + RSTEP * r + 4 * kb + i);
            if (m < 0) continue;
            E* dst = reinterpret_cast<E*>(p.out) + (size_t)m * p.N + n0 + wn * WN + j;
#pragma unroll
            for (int c = 0; c < CB; ++c) dst[16 * c] = (E)acc[r][c][i];
        }
}

// ------------------------------------------------------------------ host side

// The pipelined kernel addresses its buffers with 32-bit byte offsets and marks zero rows
// with offsets from 2^31 up, so every buffer it reads must stay below 2 GiB.
static bool dma_ok(int N, int K, int G, long long a_rows) {
    const long long lim = 1ll << 31;
    return G % BK == 0 && K % G == 0 && (long long)K * N / 2 < lim && a_rows * K * 2 < lim &&
           (long long)(K / G) * N * 2 < lim;
}

PrefillShape prefill_shape(int fmt, int M, int N, int K, int G, int num_cus, int max_ksplit) {
    PrefillShape s{};
    (void)fmt;
    if (M < 1 || N % 8 || K % BK || G % 8 || K % G) return s;
    if (dma_ok(N, K, G, M)) {
        // Tile (BM x BN) and K split from a cost model fitted to graph-replay times of the
        // pipelined kernel (AWQ, M = 2048, N = 1792 .. 14336, K = 1792 .. 14336):
        //   rounds x BM x BN x e x K / ks  +  3.2 x ks x M x N  (ks > 1: fp32 partials)
        // with rounds = ceil(tiles x ks / CUs) and e the relative time per unit of tile area:
        // 1.00 for 256 x 224 and 256 x 256 tiles, 1.15 for 256 x 128 (a third more LDS operand
        // reads per MFMA), 1.35 for 128-row tiles (half the rows per dequantised B tile). It
        // keeps every measured choice at config 3 (4096 -> 14336: 256 x 224, 231 us; 14336 ->
        // 4096: 256 x 256 with 2 splits, 231 us against 258 us for 256 x 128 unsplit) and fixes
        // the grids that left CUs idle: one GPU's share of an 8-way tensor-parallel layer,
        // M=2048, 4096 -> 1792, took 128 x 224 tiles (128 workgroups) in ~75 us, 256 x 128 with
        // 2 splits 53 us; 4096 -> 3584 128 x 224 ~85 us, 256 x 128 73 us. 256 x 192 tiles
        // (e = 1.2: a quarter of the dequantising lanes idle, narrower wave tiles) for widths
        // that 224 does not divide: N = 6144, K = 4096, M = 1024 / 2048 / 4096: 78.9 / 113.7 /
        // 229.6 us with 256 x 256 (2 splits / 1 / 1) against 68.0 / 102.4 / 203.1 us (the 192
        // workgroups of 256 x 256 at M = 2048 leave 64 CUs idle). A split keeps at least 8
        // stages of K, and 16 for 8 splits (the last workgroup of a tile sums 8 partials
        // alone): AWQ 14336 -> 4096 at M = 128 / 256 70.1 / 79.9 -> 52.2 / 70.5 us with 8
        // splits; GPTQ 4096 -> 6144 at M = 96 with 8 splits of 8 stages 38.2 us against 27.6
        // with 4. Ties go to larger tiles and fewer splits.
        double best = -1.0;
        for (int bm : {256, 128}) {
            for (int bn : {256, 224, 192, 128}) {
                if (N % bn) continue;
                if ((bn == 128 || bn == 192) && bm != 256) continue;   // 128/192-wide tiles only with 256 rows
                const double e = bm == 128 ? 1.35 : bn == 128 ? 1.15 : bn == 192 ? 1.2 : 1.0;
                const long long tiles = (long long)(N / bn) * ((M + bm - 1) / bm);
                for (int ks = 1; ks <= 8; ks *= 2) {
                    if (ks > 1 && (bm != 256 || ks > max_ksplit || (K / BK) % ks ||
                                   K / BK / ks < (ks == 8 ? 16 : 8)))
                        break;
                    const long long rounds = (tiles * ks + num_cus - 1) / num_cus;
                    const double cost = (double)rounds * bm * bn * e * ((double)K / ks) +
                                        (ks > 1 ? 3.2 * ks * (double)M * N : 0.0);
                    if (best < 0 || cost < best * (1.0 - 1e-9)) {
                        best = cost; s.bm = bm; s.bn = bn; s.ksplit = ks;
                    }
                }
            }
        }
        if (best >= 0) {
            s.dma = true;
            s.col_tiles = N / s.bn;
            s.row_tiles = (M + s.bm - 1) / s.bm;
            s.lds = prefill_dma_lds(s.bm, s.bn);
            s.ok = true;
            return s;
        }
    }
    if (N % BN) return s;
    const int col_tiles = N / BN;
    // 256-row tiles when they still give every CU a workgroup, else 128
    s.bm = ((M + 255) / 256) * col_tiles >= num_cus ? 256 : 128;
    s.bn = BN;
    s.ksplit = 1;
    s.col_tiles = col_tiles;
    s.row_tiles = (M + s.bm - 1) / s.bm;
    s.lds = (size_t)2 * (s.bm + BN) * LD * sizeof(half_t);
    s.ok = true;
    return s;
}

template <typename F>
static void allow_lds(F* kernel, size_t lds) {
    // dynamic LDS above 64 KiB must be allowed for the kernel before it is launched
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

// The dynamic-LDS allowance is set on every launch (a host-side attribute, cheap beside these
// kernels): once per process would miss other devices and race between host threads.
template <int FMT, int BM, int BN2, bool MOE, typename E = half_t>
static void launch_dma_t(const PrefillParams& p, dim3 grid, size_t lds, hipStream_t st) {
    allow_lds(&prefill_dma_kernel<FMT, BM, BN2, MOE, E>, prefill_dma_lds(BM, BN2));
    hipLaunchKernelGGL((prefill_dma_kernel<FMT, BM, BN2, MOE, E>), grid, dim3(PF_THREADS), lds, st, p);
}

template <int FMT, bool MOE, typename E = half_t>
static void launch_dma_fmt(const PrefillParams& p, int bm, int bn, dim3 grid, size_t lds,
                           hipStream_t st) {
    if constexpr (MOE) {
        if (bm == 64) launch_dma_t<FMT, 64, 256, true>(p, grid, lds, st);
        else if (bm == 128 && bn == 224) launch_dma_t<FMT, 128, 224, true>(p, grid, lds, st);
        else if (bm == 128 && bn == 128) launch_dma_t<FMT, 128, 128, true>(p, grid, lds, st);
        else if (bm == 128) launch_dma_t<FMT, 128, 256, true>(p, grid, lds, st);
        else if (bm == 192 && bn == 224) launch_dma_t<FMT, 192, 224, true>(p, grid, lds, st);
        else if (bm == 192 && bn == 128) launch_dma_t<FMT, 192, 128, true>(p, grid, lds, st);
        else if (bm == 192) launch_dma_t<FMT, 192, 256, true>(p, grid, lds, st);
        else if (bn == 224) launch_dma_t<FMT, 256, 224, true>(p, grid, lds, st);
        else if (bn == 128) launch_dma_t<FMT, 256, 128, true>(p, grid, lds, st);
        else launch_dma_t<FMT, 256, 256, true>(p, grid, lds, st);
    } else {
        if (bm == 256 && bn == 224) launch_dma_t<FMT, 256, 224, false, E>(p, grid, lds, st);
        else if (bm == 256 && bn == 192) launch_dma_t<FMT, 256, 192, false, E>(p, grid, lds, st);
        else if (bm == 256 && bn == 128) launch_dma_t<FMT, 256, 128, false, E>(p, grid, lds, st);
        else if (bm == 256) launch_dma_t<FMT, 256, 256, false, E>(p, grid, lds, st);
        else if (bn == 224) launch_dma_t<FMT, 128, 224, false, E>(p, grid, lds, st);
        else launch_dma_t<FMT, 128, 256, false, E>(p, grid, lds, st);
    }
}

template <bool MOE>
static hipError_t launch_dma_any(int fmt, const PrefillParams& p, int bm, int bn, dim3 grid,
                                 size_t lds, hipStream_t st) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (fmt == FMT_AWQ) launch_dma_fmt<FMT_AWQ, MOE>(p, bm, bn, grid, lds, st);
    else if (fmt == FMT_GPTQ) launch_dma_fmt<FMT_GPTQ, MOE>(p, bm, bn, grid, lds, st);
    else if (fmt == FMT_GPTQ_SYM) launch_dma_fmt<FMT_GPTQ_SYM, MOE>(p, bm, bn, grid, lds, st);
    else if (fmt == FMT_PREP) launch_dma_fmt<FMT_PREP, MOE>(p, bm, bn, grid, lds, st);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int FMT, int BM, bool MOE>
static void launch_t(const PrefillParams& p, dim3 grid, size_t lds, hipStream_t st) {
    // stages of loads in flight: deeper rings do not fit beside the accumulators (they end
    // up in AGPRs and every use pays an AGPR->VGPR copy)
    constexpr int D = 1;
    allow_lds(&prefill_kernel<FMT, BM, D, MOE>, lds);   // every launch, as above
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

hipError_t launch_prefill(int fmt, const PrefillParams& p, const PrefillShape& s, hipStream_t st,
                          bool bf16) {
    if (bf16) {   // the pipelined kernel on the dense checkpoint layouts only
        (void)hipGetLastError();
        if (!s.dma) return hipErrorInvalidValue;
        const dim3 grid(s.col_tiles, s.row_tiles, s.ksplit);
        if (fmt == FMT_AWQ) launch_dma_fmt<FMT_AWQ, false, bf16_t>(p, s.bm, s.bn, grid, s.lds, st);
        else if (fmt == FMT_GPTQ) launch_dma_fmt<FMT_GPTQ, false, bf16_t>(p, s.bm, s.bn, grid, s.lds, st);
        else if (fmt == FMT_GPTQ_SYM) launch_dma_fmt<FMT_GPTQ_SYM, false, bf16_t>(p, s.bm, s.bn, grid, s.lds, st);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (s.dma)
        return launch_dma_any<false>(fmt, p, s.bm, s.bn, dim3(s.col_tiles, s.row_tiles, s.ksplit),
                                     s.lds, st);
    return launch_any<false>(fmt, p, s.bm, dim3(s.col_tiles, s.row_tiles), s.lds, st);
}

bool moe_gemm_supported(int N, int K, int G, int block_m) {
    return N % BN == 0 && K % BK == 0 && G % 8 == 0 && K % G == 0 &&
           (block_m == 64 || block_m == 128);
}

bool moe_tiles_supported(int N, int K, int G, long long a_rows, int bn) {
    return (bn == 256 || bn == 224 || bn == 128) && N % bn == 0 && K % BK == 0 && G % 8 == 0 &&
           K % G == 0 && dma_ok(N, K, G, a_rows);
}

hipError_t launch_moe_gemm_tiles(int fmt, const PrefillParams& p, int tile_bm, int bn,
                                 int max_tiles, hipStream_t st) {
    const bool shape_ok = (tile_bm == 64 && bn == 256) || tile_bm == 128 || tile_bm == 192 ||
                          tile_bm == 256;
    if (!p.tiles || !p.num_tiles || !shape_ok ||
        !moe_tiles_supported(p.N, p.K, p.G, (p.num_pairs + p.a_div - 1) / p.a_div, bn))
        return hipErrorInvalidValue;
    if (p.ksplit > 1 && (!p.ws || !p.counters || (p.K / BK) % p.ksplit ||
                         (size_t)(p.N / bn) * max_tiles > SPLITK_MAX_TILES))
        return hipErrorInvalidValue;
    PrefillParams q = p;
    q.xcd_tiles = max_tiles;   // XCD-grouped order (xcd_tile_of_block) over a 1-D grid
    const int gyp = (max_tiles + 7) & ~7;
    return launch_dma_any<true>(fmt, q, tile_bm, bn,
                                dim3((p.N / bn) * gyp * max(p.ksplit, 1)),
                                prefill_dma_lds(tile_bm, bn), st);
}

hipError_t launch_moe_gemm(int fmt, const PrefillParams& p, int block_m, int max_blocks,
                           hipStream_t st) {
    const long long a_rows = (p.num_pairs + p.a_div - 1) / p.a_div;
    if (dma_ok(p.N, p.K, p.G, a_rows) && (long long)p.K * p.N / 2 < (1ll << 31))
        return launch_dma_any<true>(fmt, p, block_m, BN, dim3(p.N / BN, max_blocks),
                                    prefill_dma_lds(block_m, BN), st);
    const size_t lds = (size_t)2 * (block_m + BN) * LD * sizeof(half_t);
    return launch_any<true>(fmt, p, block_m, dim3(p.N / BN, max_blocks), lds, st);
}

}  // namespace w4a16
