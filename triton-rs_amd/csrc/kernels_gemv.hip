// Decode-regime W4A16 GEMV (M <= 8): HBM-bound.
//
// Computes out[m, n] = sum_k x[m, k] * W16[k, n] for the reference's two packings
// (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:15-32 GPTQ [K/8, N] packed along K;
// awq_gemm_int4_typed.rs:10-31 AWQ [K, N/8] packed along N, slot order [0,4,1,5,2,6,3,7]),
// split over K so that a launch has ~900 workgroups, with a deterministic in-kernel
// split-K hand-off (splitk.h: the workgroup that arrives last at the tile's counter sums
// the fp32 partials in split order). At M = 1 all splits of a tile run on one XCD and the
// hand-off stays in that XCD's L2.
//
// VALU kernels (AWQ M = 1, GPTQ M <= 4): per lane the inner loop is 128-bit (or 32-bit)
// coalesced loads of packed words, a nibble unpack into fp16 with the 0x6400 exponent
// trick (1024 + q, or 1024 + 16 q for the odd nibble of each byte, so no shift is needed
// for it), and v_dot2c_f32_f16 against pairs of x. No MFMA. All rows a lane touches lie
// in one quantisation group, so the zero point and the scale are applied once per lane
// and column to the fp32 sum:
//     sum_k x_k (q_k - z) s = s * (A - 1024 X - z X),   A = sum_k x_k (1024 + q_k)
// which equals the reference's dequant-then-dot up to fp32 rounding (the reference rounds
// each dequantised weight to fp16 first; the difference is < 2^-11 relative per term).
// The AWQ matrix-core kernel (M = 2..8) moves the dot products to v_mfma (below).
#include <type_traits>

#include "device_common.h"
#include "launch.h"
#include "splitk.h"

namespace w4a16 {

// ------------------------------------------------------------------ AWQ GEMV

// Tile: 256 columns (32 words per row) x R rows. Lane mapping: LPR = 32 / CW lanes per row,
// each owning CW words (8*CW columns); RPW = 64 / LPR row-lanes per wave; a lane walks RL
// consecutive rows (all in one group: G % RL == 0).
//
// Load order per wave: x (small, cache-resident after first use), then the RL weight rows
// (non-temporal buffer loads: one per-lane offset, the row offset in an SGPR), then the
// group's scales and zero words (non-temporal). Loads complete in issue order, so the weights
// are consumed while the scales are still in flight; issued first, the scattered scale and
// zero requests cost 0.3 us at K=4096, N=14336 (7.93 vs 8.28 us, same kernel otherwise), and
// cached rather than streamed 0.2 us more. The scheduling barriers keep this order.
// E: the element type of x, the scales and the output. bf16 unpacks 128 + q (every nibble
// shifted to bits 0..3) and accumulates with v_dot2c_f32_bf16: s * (A - 128 X - z X).
template <int M, int CW, int RL, int WAVES, bool XCD, bool FIX, typename E = half_t>
__global__ void __launch_bounds__(64 * WAVES)
gemv_awq_kernel(GemvParams p) {
    constexpr bool BF = std::is_same<E, bf16_t>::value;
    typedef typename pair2<E>::type e2_t;
    constexpr int LPR = 32 / CW;
    constexpr int RPW = 64 / LPR;
    constexpr int RB = RPW * WAVES;
    constexpr int R = RB * RL;
    constexpr int C = 256;
    static_assert(RL % 2 == 0 && RL % 8 == 0, "rows per lane must be a multiple of 8");
    static_assert(CW == 1 || CW == 2 || CW == 4, "words per lane");

    __shared__ float red[RB][M][C];
    __shared__ int flag;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int cl = lane % LPR;
    const int rb = wave * RPW + lane / LPR;
    int ct, split;
    tile_of_block<XCD>(p.col_tiles, p.splits, ct, split);
    constexpr int SC = XCD ? SCOPE_XCD : SCOPE_DEVICE;
    const int NW = p.N >> 3;                       // words per qweight row
    const int wc0 = ct * 32 + cl * CW;             // first word column of this lane
    const int kw = split * R + wave * RPW * RL;    // first row of the wave (uniform)
    const int k0 = kw + (lane / LPR) * RL;         // first row of this lane
    const int g = k0 / p.G;

    // ---- x pairs (rows 2i, 2i+1 of this lane) for every m, and X = sum of x
    e2_t xs[M][RL / 2];
    float X[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint4* xp = reinterpret_cast<const uint4*>(p.x + (size_t)m * p.K + k0);
#pragma unroll
        for (int i = 0; i < RL / 8; ++i) {
            const uint4 v = xp[i];
            xs[m][4 * i + 0] = as_pair<E>(v.x); xs[m][4 * i + 1] = as_pair<E>(v.y);
            xs[m][4 * i + 2] = as_pair<E>(v.z); xs[m][4 * i + 3] = as_pair<E>(v.w);
        }
    }

    // ---- all weight rows of the lane, then its scales and zero words
    uint32_t w[RL][CW];
    const bufrsrc_t wr = make_rsrc(p.qweight, (uint32_t)((size_t)p.K * p.N / 2));
    const uint32_t voff = ((uint32_t)(lane / LPR) * (uint32_t)RL * (uint32_t)NW + (uint32_t)wc0) * 4u;
    const uint32_t row_bytes = (uint32_t)NW * 4u;
    const uint32_t soff0 = (uint32_t)kw * row_bytes;
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const uint32_t so = soff0 + (uint32_t)j * row_bytes;
        if constexpr (CW == 4) {
            const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, so, 2));
            w[j][0] = v.x; w[j][1] = v.y; w[j][2] = v.z; w[j][3] = v.w;
        } else if constexpr (CW == 2) {
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, voff, so, 2));
            w[j][0] = v.x; w[j][1] = v.y;
        } else {
            w[j][0] = buf_ld_stream(wr, voff, so);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t qz[CW];
    u32x4 sv[CW];
#pragma unroll
    for (int c = 0; c < CW; ++c) {
        qz[c] = p.qzeros ? __builtin_nontemporal_load(p.qzeros + (size_t)g * NW + wc0 + c) : 0u;
        sv[c] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(p.scales + (size_t)g * p.N + 8 * (wc0 + c)));
    }
    __builtin_amdgcn_sched_barrier(0);
    float XB[M];   // the exponent trick's bias (1024 or 128) times X
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float sx = 0.f;
        const e2_t one2 = {(E)1.0f, (E)1.0f};
#pragma unroll
        for (int i = 0; i < RL / 2; ++i) sx = dot2(xs[m][i], one2, sx);
        X[m] = sx;
        XB[m] = pair2<E>::bias * sx;
    }

    // ---- main loop: acc[m][cw][slot]
    float acc[M][CW][8];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int s = 0; s < 8; ++s) acc[m][c][s] = 0.f;

#pragma unroll
    for (int i = 0; i < RL / 2; ++i) {
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            const uint32_t a = w[2 * i][c], b = w[2 * i + 1][c];
            // bytes {a0,a1,b0,b1}: slots 0-3 of row 2i in the low half, of row 2i+1 in the high
            const uint32_t lo = perm(b, a, 0x05040100u);
            const uint32_t hi = perm(b, a, 0x07060302u);
            const uint32_t lo8 = lo >> 8, hi8 = hi >> 8;
            e2_t h[8];
            if constexpr (BF) {       // slot s: 128 + q
                h[0] = nib_pair_bf16(lo);       h[1] = nib_pair_bf16(lo >> 4);
                h[2] = nib_pair_bf16(lo8);      h[3] = nib_pair_bf16(lo8 >> 4);
                h[4] = nib_pair_bf16(hi);       h[5] = nib_pair_bf16(hi >> 4);
                h[6] = nib_pair_bf16(hi8);      h[7] = nib_pair_bf16(hi8 >> 4);
            } else {
                h[0] = nib_pair(lo);      // slot 0: 1024 + q
                h[1] = nib_pair16(lo);    // slot 1: 1024 + 16 q
                h[2] = nib_pair(lo8);     // slot 2
                h[3] = nib_pair16(lo8);   // slot 3 (x16)
                h[4] = nib_pair(hi);      // slot 4
                h[5] = nib_pair16(hi);    // slot 5 (x16)
                h[6] = nib_pair(hi8);     // slot 6
                h[7] = nib_pair16(hi8);   // slot 7 (x16)
            }
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int s = 0; s < 8; ++s) acc[m][c][s] = dot2(h[s], xs[m][i], acc[m][c][s]);
        }
    }

    // ---- zero point and scale, once per lane and column; columns written in natural order
#pragma unroll
    for (int c = 0; c < CW; ++c) {
        const E* sh = reinterpret_cast<const E*>(&sv[c]);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float col[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int n = awq_col_of_slot(s);
                const float z = (float)nib(qz[c], s);
                // fp16: odd slots were unpacked as 1024 + 16 q
                const float u = (!BF && (s & 1)) ? __builtin_fmaf(acc[m][c][s] - XB[m], 1.0f / 16.0f, -z * X[m])
                                                 : acc[m][c][s] - XB[m] - z * X[m];
                col[n] = (float)sh[n] * u;
            }
            float4* dst = reinterpret_cast<float4*>(&red[rb][m][(cl * CW + c) * 8]);
            dst[0] = make_float4(col[0], col[1], col[2], col[3]);
            dst[1] = make_float4(col[4], col[5], col[6], col[7]);
        }
    }
    __syncthreads();

    // ---- reduce over row blocks; write partial (or the output when there is one split)
    const int n0 = ct * C;
    if constexpr (FIX) {   // fixed-point hand-off (splitk.h): one atomic per entry, no reload
        constexpr int T = 64 * WAVES, NE = (M * C + T - 1) / T;
        size_t off[NE];
        float v[NE];
        int n = 0;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int i = (int)threadIdx.x + e * T;
            if (i >= M * C) break;
            const int m = i / C, cidx = i - m * C;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < RB; ++r) s += red[r][m][cidx];
            off[e] = (size_t)m * p.N + n0 + cidx;
            v[e] = s;
            n = e + 1;
        }
        splitk_fixed_commit<SC, NE, E>(p.slots, p.masks, p.ws, (size_t)M * p.N, reinterpret_cast<E*>(p.out),
                                       off, v, n, split, p.splits);
        return;
    } else {
    for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
        const int m = i / C, cidx = i - m * C;
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < RB; ++r) s += red[r][m][cidx];
        const size_t off = (size_t)m * p.N + n0 + cidx;
        if (p.splits == 1) reinterpret_cast<E*>(p.out)[off] = (E)s;
        else st_partial<SC>(p.ws + (size_t)split * M * p.N + off, s);
    }
    if (p.splits == 1) return;
    if (splitk_arrive(splitk_counter(p.counters, ct), p.splits, &flag))
        splitk_finish<M, SC, E>(p.ws, reinterpret_cast<E*>(p.out), p.splits, p.N, n0, C);
    }
}

// ------------------------------------------------------------------ GPTQ GEMV

// Tile: C = LPR * CW columns x R k-rows. A lane owns CW consecutive columns (one 128-bit
// load per packed row for CW = 4) and RL consecutive packed rows (8*RL k, one group).
// E: as for the AWQ kernel (bf16: every nibble at bits 0..3, bias 128).
template <int FMT, int M, int CW, int RL, int WAVES, int LPR, bool XCD, bool FIX, typename E = half_t>
__global__ void __launch_bounds__(64 * WAVES)
gemv_gptq_kernel(GemvParams p) {
    constexpr bool BF = std::is_same<E, bf16_t>::value;
    typedef typename pair2<E>::type e2_t;
    constexpr int RPW = 64 / LPR;
    constexpr int RB = RPW * WAVES;
    constexpr int C = LPR * CW;
    constexpr int RK = RB * RL * 8;  // k rows per block

    __shared__ float red[RB][M][C];
    __shared__ int flag;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cl = lane % LPR;
    const int rb = wave * RPW + lane / LPR;
    int ct, split;
    tile_of_block<XCD>(p.col_tiles, p.splits, ct, split);
    constexpr int SC = XCD ? SCOPE_XCD : SCOPE_DEVICE;
    const int n0 = ct * C;
    const int c0 = n0 + cl * CW;                       // first column of this lane
    const int kp0 = (split * RK) / 8 + rb * RL;        // first packed row
    const int k0 = kp0 * 8;
    const int g = k0 / p.G;

    // x for packed row j, rearranged to the unpack order: (x0,x4) (x1,x5) (x2,x6) (x3,x7)
    e2_t xs[M][RL][4];
    float X[M], B[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float x1 = 0.f, x16 = 0.f;
        const e2_t one2 = {(E)1.0f, (E)1.0f};
#pragma unroll
        for (int j = 0; j < RL; ++j) {
            const uint4 v = *reinterpret_cast<const uint4*>(p.x + (size_t)m * p.K + k0 + 8 * j);
            xs[m][j][0] = as_pair<E>(perm(v.z, v.x, 0x05040100u));
            xs[m][j][1] = as_pair<E>(perm(v.z, v.x, 0x07060302u));
            xs[m][j][2] = as_pair<E>(perm(v.w, v.y, 0x05040100u));
            xs[m][j][3] = as_pair<E>(perm(v.w, v.y, 0x07060302u));
            x1 = dot2(xs[m][j][0], one2, x1);
            x1 = dot2(xs[m][j][2], one2, x1);
            x16 = dot2(xs[m][j][1], one2, x16);
            x16 = dot2(xs[m][j][3], one2, x16);
        }
        X[m] = x1 + x16;
        B[m] = BF ? 128.0f * X[m] : 1024.0f * (x1 + x16 * (1.0f / 16.0f));
    }

    uint32_t w[RL][CW];
    const uint32_t off0 = (uint32_t)kp0 * (uint32_t)p.N + (uint32_t)c0;
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const uint32_t off = off0 + (uint32_t)j * (uint32_t)p.N;
        if constexpr (CW == 4) {
            const u32x4 v = ld_stream4(at_bytes(p.qweight, 4u * off));
            w[j][0] = v.x; w[j][1] = v.y; w[j][2] = v.z; w[j][3] = v.w;
        } else if constexpr (CW == 2) {
            const u32x2 v = ld_stream2(at_bytes(p.qweight, 4u * off));
            w[j][0] = v.x; w[j][1] = v.y;
        } else {
            w[j][0] = ld_stream(at_bytes(p.qweight, 4u * off));
        }
    }

    float a1[M][CW], a16[M][CW];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int c = 0; c < CW; ++c) { a1[m][c] = 0.f; a16[m][c] = 0.f; }

#pragma unroll
    for (int j = 0; j < RL; ++j) {
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            const uint32_t q = w[j][c];
            const uint32_t q8 = q >> 8;
            e2_t h0, h1, h2, h3;
            if constexpr (BF) {
                h0 = nib_pair_bf16(q);   h1 = nib_pair_bf16(q >> 4);     // (k0, k4), (k1, k5)
                h2 = nib_pair_bf16(q8);  h3 = nib_pair_bf16(q8 >> 4);    // (k2, k6), (k3, k7)
            } else {
                h0 = nib_pair(q);      // k0, k4
                h1 = nib_pair16(q);    // k1, k5 (x16)
                h2 = nib_pair(q8);     // k2, k6
                h3 = nib_pair16(q8);   // k3, k7 (x16)
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                a1[m][c] = dot2(h0, xs[m][j][0], a1[m][c]);
                a1[m][c] = dot2(h2, xs[m][j][2], a1[m][c]);
                a16[m][c] = dot2(h1, xs[m][j][1], a16[m][c]);
                a16[m][c] = dot2(h3, xs[m][j][3], a16[m][c]);
            }
        }
    }

    // zero point and scale for the lane's CW columns (same qzeros word: CW divides 8)
    uint32_t qz = 0;
    if constexpr (FMT == FMT_GPTQ) qz = p.qzeros[(size_t)g * (p.N >> 3) + (c0 >> 3)];
    E sc[CW];
    const E* scales = reinterpret_cast<const E*>(p.scales);
    if constexpr (CW == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(scales + (size_t)g * p.N + c0);
        const E* hv = reinterpret_cast<const E*>(&v);
#pragma unroll
        for (int c = 0; c < 4; ++c) sc[c] = hv[c];
    } else {
#pragma unroll
        for (int c = 0; c < CW; ++c) sc[c] = scales[(size_t)g * p.N + c0 + c];
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            const float z = (float)zero_of<FMT>(qz, c0 + c, p.zero_offset);
            const float u = a1[m][c] + a16[m][c] * (BF ? 1.0f : 1.0f / 16.0f) - B[m] - z * X[m];
            red[rb][m][cl * CW + c] = (float)sc[c] * u;
        }
    }
    __syncthreads();

    if constexpr (FIX) {   // fixed-point hand-off (splitk.h): one atomic per entry, no reload
        constexpr int T = 64 * WAVES, NE = (M * C + T - 1) / T;
        size_t off[NE];
        float v[NE];
        int n = 0;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int i = (int)threadIdx.x + e * T;
            if (i >= M * C) break;
            const int m = i / C, cidx = i - m * C;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < RB; ++r) s += red[r][m][cidx];
            off[e] = (size_t)m * p.N + n0 + cidx;
            v[e] = s;
            n = e + 1;
        }
        splitk_fixed_commit<SC, NE, E>(p.slots, p.masks, p.ws, (size_t)M * p.N, reinterpret_cast<E*>(p.out),
                                       off, v, n, split, p.splits);
        return;
    } else {
    for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
        const int m = i / C, cidx = i - m * C;
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < RB; ++r) s += red[r][m][cidx];
        const size_t off = (size_t)m * p.N + n0 + cidx;
        if (p.splits == 1) reinterpret_cast<E*>(p.out)[off] = (E)s;
        else st_partial<SC>(p.ws + (size_t)split * M * p.N + off, s);
    }
    if (p.splits == 1) return;
    if (splitk_arrive(splitk_counter(p.counters, ct), p.splits, &flag))
        splitk_finish<M, SC, E>(p.ws, reinterpret_cast<E*>(p.out), p.splits, p.N, n0, C);
    }
}

// ------------------------------------------------------------------ AWQ, M = 5..8: matrix-core dot

// For 5 <= M <= 8 the VALU dot products above would cost M dot2 per nibble pair. Here the
// dot products run on v_mfma_f32_16x16x32_f16 and the vector ALUs only unpack. An AWQ word
// holds 8 columns of one row while the MFMA B operand wants 8 k of one column per lane, so
// instead of transposing nibbles the MFMA contraction index is made (row, nibble class) and
// the A operand carries x block-diagonally:
//   lane (j, q) of B supplies, for word column j of its row r_q, the 8 values
//     e = 0..7: fp16(1024 + c_e q[slot(e)]), slot = [0,4,1,5,2,6,3,7][e], c_e in {1, 16}
//     (v_and_or_b32 of w and w >> 8 with 0x000F000F / 0x00F000F0 and the 0x6400 exponent);
//   lane (i, q) of A supplies x[m][r_q] at element e = i % 8 (m = 2 set + i / 8), else 0.
// Then D[8 (m % 2) + e][j] = sum_q x[m][r_q] (1024 + c_e q[r_q][slot(e)]): one MFMA covers 4
// rows x 16 words x 8 slots for two rows of x. After the wave's R rows (one quantisation
// group) the zero and scale are applied once, as in the kernel above:
//   sum_k x_k (q_k - z) s = s ((A - 1024 X) / c - z X).
// Per 8 weights: one shift and four v_and_or_b32; per step and pair of x rows four
// v_perm_b32 place x into A.
//
// Tile: WW = 16 CW words (8 WW columns) x WAVES * R rows; lane (j, q) streams rows
// r0 + (R/4) q + s, s = 0 .. R/4 - 1, of word columns CW j .. CW j + CW - 1 with PF steps of
// loads in flight.
template <int M, int CW, int R, int WAVES, int PF, bool XCD, bool FIX>
__global__ void __launch_bounds__(64 * WAVES)
gemv_awq_mfma_kernel(GemvParams p) {
    constexpr int S = R / 4;          // steps per wave
    constexpr int MS = (M + 1) / 2;   // MFMA sets: two rows of x each
    constexpr int WW = 16 * CW;       // words per tile row
    constexpr int C = 8 * WW;         // columns per tile
    static_assert(S % 8 == 0 && PF <= S && (CW == 2 || CW == 4), "tile shape");
    static_assert(64 * WAVES <= FINISH_MAX_THREADS, "split-K finish buffer");

    __shared__ float red[WAVES][M][C];
    __shared__ int flag;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, q = lane >> 4;
    int ct, split;
    tile_of_block<XCD>(p.col_tiles, p.splits, ct, split);
    constexpr int SC = XCD ? SCOPE_XCD : SCOPE_DEVICE;
    const int NW = p.N >> 3;
    const int wc = ct * WW + CW * j;                   // first word column of this lane
    const int rw0 = (split * WAVES + wave) * R;        // first row of this wave
    const int rl0 = rw0 + S * q;                       // rows of this lane: rl0 + s
    const int g = rw0 / p.G;

    // ---- weight ring: step s of the lane lives in slot s % PF
    uint32_t bw[PF][CW];
    const uint32_t off0 = (uint32_t)rl0 * (uint32_t)NW + (uint32_t)wc;
    auto issue = [&](int u, int s) {
        const uint32_t off = off0 + (uint32_t)s * (uint32_t)NW;
        if constexpr (CW == 4) {
            const u32x4 v = ld_stream4(at_bytes(p.qweight, 4u * off));
            bw[u][0] = v.x; bw[u][1] = v.y; bw[u][2] = v.z; bw[u][3] = v.w;
        } else {
            const u32x2 v = ld_stream2(at_bytes(p.qweight, 4u * off));
            bw[u][0] = v.x; bw[u][1] = v.y;
        }
    };
#pragma unroll
    for (int u = 0; u < PF; ++u) issue(u, u);

    // ---- x of the lane's rows for its A row (m = 2 ms + j / 8), S halfs per set
    uint32_t xr[MS][S / 2];
    float xsum[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int m = 2 * ms + (j >> 3);
        xsum[ms] = 0.f;
        if (m < M) {
            const u32x4* xp = reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.K + rl0);
#pragma unroll
            for (int h = 0; h < S / 8; ++h) {
                const u32x4 v = xp[h];
                xr[ms][4 * h + 0] = v.x; xr[ms][4 * h + 1] = v.y;
                xr[ms][4 * h + 2] = v.z; xr[ms][4 * h + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int h = 0; h < S / 2; ++h) xr[ms][h] = 0u;
        }
        const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
        for (int h = 0; h < S / 2; ++h) xsum[ms] = dot2(as_h2(xr[ms][h]), one2, xsum[ms]);
    }
    // v_perm_b32 selectors placing half (s % 2) of an x word at element e = j % 8 of the A
    // operand (selector byte 0x0C yields zero)
    uint32_t sel[2][4];
    {
        const int e = j & 7;
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            const uint32_t b0 = 2u * par, b1 = b0 + 1u;
            const uint32_t half_sel = (e & 1) ? ((b1 << 24) | (b0 << 16) | 0x0C0Cu)
                                              : (0x0C0C0000u | (b1 << 8) | b0);
#pragma unroll
            for (int t = 0; t < 4; ++t) sel[par][t] = (t == (e >> 1)) ? half_sel : 0x0C0C0C0Cu;
        }
    }

    float4_t acc[MS][CW];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[ms][c] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s0 = 0; s0 < S; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int s = s0 + u;
            half8_t af[MS];
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const uint32_t xw = xr[ms][s >> 1];
                const u32x4 a = {perm(xw, xw, sel[s & 1][0]), perm(xw, xw, sel[s & 1][1]),
                                 perm(xw, xw, sel[s & 1][2]), perm(xw, xw, sel[s & 1][3])};
                af[ms] = __builtin_bit_cast(half8_t, a);
            }
#pragma unroll
            for (int c = 0; c < CW; ++c) {
                const uint32_t w = bw[u][c], w8 = w >> 8;
                const u32x4 b = {as_u32(nib_pair(w)), as_u32(nib_pair16(w)), as_u32(nib_pair(w8)),
                                 as_u32(nib_pair16(w8))};
                const half8_t bf = __builtin_bit_cast(half8_t, b);
#pragma unroll
                for (int ms = 0; ms < MS; ++ms)
                    acc[ms][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[ms], bf, acc[ms][c], 0, 0, 0);
            }
            if (s + PF < S) issue(u, s + PF);
        }
    }

    // ---- lane (j, q) holds D rows 4 q .. 4 q + 3 of each set: m = 2 ms + q / 2, classes
    // e = 4 (q % 2) + r, i.e. columns 4 (q % 2) + r of its words
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        float tsum = xsum[ms];
        tsum += __shfl_xor(tsum, 16);
        tsum += __shfl_xor(tsum, 32);
        xsum[ms] = __shfl(tsum, 8 * (q >> 1));
    }
    const int hq = q & 1;
#pragma unroll
    for (int c = 0; c < CW; ++c) {
        const int word = wc + c;
        const uint32_t qz = p.qzeros[(size_t)g * NW + word];
        const u32x2 sv = *reinterpret_cast<const u32x2*>(p.scales + (size_t)g * p.N + 8 * word + 4 * hq);
        const half2_t s01 = as_h2(sv.x), s23 = as_h2(sv.y);
        const float scl[4] = {(float)s01.x, (float)s01.y, (float)s23.x, (float)s23.y};
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int m = 2 * ms + (q >> 1);
            if (m >= M) continue;
            const float X = xsum[ms];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int col = 4 * hq + r;                 // column within the word
                const float z = (float)nib(qz, awq_slot(col));
                const float inv_c = (r & 2) ? (1.0f / 16.0f) : 1.0f;
                const float u = (acc[ms][c][r] - 1024.0f * X) * inv_c - z * X;
                red[wave][m][8 * (CW * j + c) + col] = scl[r] * u;
            }
        }
    }
    __syncthreads();

    // ---- reduce over waves; write partial (or the output when there is one split)
    const int n0 = ct * C;
    if constexpr (FIX) {   // fixed-point hand-off (splitk.h): one atomic per entry, no reload
        constexpr int T = 64 * WAVES, E = (M * C + T - 1) / T;
        size_t off[E];
        float v[E];
        int n = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = (int)threadIdx.x + e * T;
            if (i >= M * C) break;
            const int m = i / C, cidx = i - m * C;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) s += red[w][m][cidx];
            off[e] = (size_t)m * p.N + n0 + cidx;
            v[e] = s;
            n = e + 1;
        }
        splitk_fixed_commit<SC, E>(p.slots, p.masks, p.ws, (size_t)M * p.N, p.out, off, v, n, split, p.splits);
        return;
    } else {
    for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
        const int m = i / C, cidx = i - m * C;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += red[w][m][cidx];
        const size_t off = (size_t)m * p.N + n0 + cidx;
        if (p.splits == 1) p.out[off] = (half_t)sum;
        else st_partial<SC>(p.ws + (size_t)split * M * p.N + off, sum);
    }
    if (p.splits == 1) return;
    if (splitk_arrive(splitk_counter(p.counters, ct), p.splits, &flag))
        splitk_finish<M, SC>(p.ws, p.out, p.splits, p.N, n0, C);
    }
}

// ------------------------------------------------------------------ AWQ, M = 3..8: matrix cores, row-paired B

// The kernel above makes the MFMA contraction index (row, nibble class), so its A operand
// carries x block-diagonally and one MFMA does 1/8 useful work; at M = 8 the matrix cores
// are its bottleneck. Here B holds 8 consecutive rows of one column, as a GEMM wants: the
// bytes of two AWQ words (rows 2i, 2i+1) are paired with v_perm_b32 and each v_and_or_b32
// (0x6400 exponent) yields the fp16 pair (1024 + q[2i][slot], 1024 + q[2i+1][slot]) (or
// 1024 + 16 q for the odd slots, left in place), so per 16 weights: 2 perms, 2 shifts, 8
// and_or. A is x itself (rows 0..M-1 of the 16; higher rows repeat row M-1 and their D rows
// are never stored), so one MFMA does M/16 useful work. Zero point and scale are applied
// once per wave, as in the VALU kernel: s * ((D - 1024 X) / c - z X).
//
// Tile: 256 columns (32 words) x 128 W rows; wave w owns rows 128 w .. 128 w + 127 (one
// quantisation group: G % 128 == 0). Lane (jw, kg) = (lane % 16, lane / 16) loads words
// 2 jw, 2 jw + 1 (one 64-bit load) of rows 32 b + 8 kg + i, b = 0..3, i = 0..7: all 32 loads
// of the wave in flight at once. MFMA (c, s), c = word of the pair, s = slot: B lane (jw,
// kg) = rows 8 kg .. 8 kg + 7 of block b, column of word 2 jw + c in slot s; A lane (m, kg) =
// x[min(m, M - 1)][rows 8 kg .. 8 kg + 7 of block b]. D lane (jw, kg) holds rows 4 kg + i.
// Measured against gemv_awq_mfma_kernel (graph replays, 20 rotated weight sets): K=4096 ->
// N=14336 M=3/4/5/8: 10.9/10.3/13.3/14.4 -> 9.4/9.7/10.8/11.3 us; K=14336 -> N=4096 M=4/8:
// 10.2/15.6 -> 9.7/12.4 us; at M = 2 (8.4 vs 9.0 us) and M = 1 the other kernels stay.
// E: the element type (bf16: 128 + q with every nibble shifted to bits 0..3, bf16 MFMA).
template <int M, int W, bool FIX, typename E = half_t>
__global__ void __launch_bounds__(64 * W)
gemv_awq_rows_kernel(GemvParams p) {
    constexpr bool BF = std::is_same<E, bf16_t>::value;
    typedef typename pair2<E>::type e2_t;
    typedef typename vec8<E>::type v8_t;
    constexpr int C = 256;
    constexpr int SC = SCOPE_DEVICE;
    static_assert(64 * W <= FINISH_MAX_THREADS, "split-K finish buffer");
    __shared__ float red[W][M][C];
    __shared__ int flag;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int jw = lane & 15, kg = lane >> 4;
    const int ct = blockIdx.x, split = blockIdx.y;
    const int NW = p.N >> 3;
    const int r0 = (split * W + wave) * 128;       // first row of the wave
    const int g = r0 / p.G;

    // ---- x of the wave's rows for A row min(jw, M - 1), then the 32 weight loads, then the
    // group's scales and zero words (loads complete in issue order)
    const int mx = min(jw, M - 1);
    u32x4 xv[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
        xv[b] = *reinterpret_cast<const u32x4*>(p.x + (size_t)mx * p.K + r0 + 32 * b + 8 * kg);
    const bufrsrc_t wr = make_rsrc(p.qweight, (uint32_t)((size_t)p.K * p.N / 2));
    const uint32_t voff = ((uint32_t)(8 * kg) * (uint32_t)NW + (uint32_t)(ct * 32 + 2 * jw)) * 4u;
    const uint32_t row_bytes = (uint32_t)NW * 4u;
    u32x2 w[4][8];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[b][i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                          wr, voff, (uint32_t)(r0 + 32 * b + i) * row_bytes, 2));
    __builtin_amdgcn_sched_barrier(0);
    uint32_t qz[2];
    u32x4 sv[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int word = ct * 32 + 2 * jw + c;
        qz[c] = __builtin_nontemporal_load(p.qzeros + (size_t)g * NW + word);
        sv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.scales + (size_t)g * p.N + 8 * word));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- main loop: 16 MFMAs per 32 rows
    float4_t acc[2][8];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[c][s] = float4_t{0.f, 0.f, 0.f, 0.f};
    float xs = 0.f;
    const e2_t one2 = {(E)1.0f, (E)1.0f};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const v8_t xa = __builtin_bit_cast(v8_t, xv[b]);
        xs = dot2(as_pair<E>(xv[b].x), one2, xs); xs = dot2(as_pair<E>(xv[b].y), one2, xs);
        xs = dot2(as_pair<E>(xv[b].z), one2, xs); xs = dot2(as_pair<E>(xv[b].w), one2, xs);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            uint32_t h[4][8];
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const uint32_t a = c ? w[b][2 * i2].y : w[b][2 * i2].x;
                const uint32_t bb = c ? w[b][2 * i2 + 1].y : w[b][2 * i2 + 1].x;
                // bytes {a0, a1, b0, b1} and {a2, a3, b2, b3}: slots 0-3 / 4-7 of the two rows
                const uint32_t lo = perm(bb, a, 0x05040100u), hi = perm(bb, a, 0x07060302u);
                const uint32_t lo8 = lo >> 8, hi8 = hi >> 8;
                if constexpr (BF) {
                    auto bp = [](uint32_t v) { return __builtin_bit_cast(uint32_t, nib_pair_bf16(v)); };
                    h[i2][0] = bp(lo);   h[i2][1] = bp(lo >> 4);  h[i2][2] = bp(lo8);  h[i2][3] = bp(lo8 >> 4);
                    h[i2][4] = bp(hi);   h[i2][5] = bp(hi >> 4);  h[i2][6] = bp(hi8);  h[i2][7] = bp(hi8 >> 4);
                } else {
                    h[i2][0] = as_u32(nib_pair(lo));   h[i2][1] = as_u32(nib_pair16(lo));
                    h[i2][2] = as_u32(nib_pair(lo8));  h[i2][3] = as_u32(nib_pair16(lo8));
                    h[i2][4] = as_u32(nib_pair(hi));   h[i2][5] = as_u32(nib_pair16(hi));
                    h[i2][6] = as_u32(nib_pair(hi8));  h[i2][7] = as_u32(nib_pair16(hi8));
                }
            }
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const u32x4 bv = {h[0][s], h[1][s], h[2][s], h[3][s]};
                acc[c][s] = mfma16x16x32(xa, __builtin_bit_cast(v8_t, bv), acc[c][s]);
            }
        }
    }

    // ---- X[m] = sum of x over the wave's rows for m = lane % 16, then for the lane's D rows
    xs += __shfl_xor(xs, 16);
    xs += __shfl_xor(xs, 32);
    float Xr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) Xr[i] = __shfl(xs, 4 * kg + i);
    // ---- zero point and scale; D row 4 kg + i, column of word 2 jw + c in slot s
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * kg + i;
        if (m >= M) continue;
        const float X = Xr[i], XB = pair2<E>::bias * Xr[i];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const E* sh = reinterpret_cast<const E*>(&sv[c]);
            float col[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int n = awq_col_of_slot(s);
                const float z = (float)nib(qz[c], s);
                // fp16: odd slots were unpacked as 1024 + 16 q
                const float u = (!BF && (s & 1)) ? __builtin_fmaf(acc[c][s][i] - XB, 1.0f / 16.0f, -z * X)
                                                 : acc[c][s][i] - XB - z * X;
                col[n] = (float)sh[n] * u;
            }
            float4* dst = reinterpret_cast<float4*>(&red[wave][m][8 * (2 * jw + c)]);
            dst[0] = make_float4(col[0], col[1], col[2], col[3]);
            dst[1] = make_float4(col[4], col[5], col[6], col[7]);
        }
    }
    __syncthreads();

    // ---- reduce over waves; split-K hand-off
    const int n0 = ct * C;
    if constexpr (FIX) {   // fixed-point hand-off (splitk.h): one atomic per entry, no reload
        constexpr int T = 64 * W, NE = (M * C + T - 1) / T;
        size_t off[NE];
        float v[NE];
        int n = 0;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int i = (int)threadIdx.x + e * T;
            if (i >= M * C) break;
            const int m = i / C, cidx = i - m * C;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < W; ++r) s += red[r][m][cidx];
            off[e] = (size_t)m * p.N + n0 + cidx;
            v[e] = s;
            n = e + 1;
        }
        splitk_fixed_commit<SC, NE, E>(p.slots, p.masks, p.ws, (size_t)M * p.N, reinterpret_cast<E*>(p.out),
                                       off, v, n, split, p.splits);
    } else {
        for (int i = threadIdx.x; i < M * C; i += blockDim.x) {
            const int m = i / C, cidx = i - m * C;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < W; ++r) s += red[r][m][cidx];
            const size_t off = (size_t)m * p.N + n0 + cidx;
            if (p.splits == 1) reinterpret_cast<E*>(p.out)[off] = (E)s;
            else st_partial<SC>(p.ws + (size_t)split * M * p.N + off, s);
        }
        if (p.splits == 1) return;
        if (splitk_arrive(splitk_counter(p.counters, ct), p.splits, &flag))
            splitk_finish<M, SC, E>(p.ws, reinterpret_cast<E*>(p.out), p.splits, p.N, n0, C);
    }
}

// ------------------------------------------------------------------ host launchers

namespace {
// AWQ: CW = 1 word per lane per row, 32 rows per lane, 4 waves -> 256 columns x 256 rows.
constexpr int AWQ_CW = 1, AWQ_RL = 32, AWQ_WAVES = 4;
constexpr int AWQ_ROWS = (64 / (32 / AWQ_CW)) * AWQ_WAVES * AWQ_RL;
// At M = 1, 8 waves (512 rows, half the splits) where K allows: 8.51 -> 8.41 us at
// K=4096, N=14336 with the fixed-point hand-off.
constexpr int AWQ_WAVES_DEEP = 8;
constexpr int AWQ_ROWS_DEEP = (64 / (32 / AWQ_CW)) * AWQ_WAVES_DEEP * AWQ_RL;
// GPTQ: CW = 4 columns per lane, 4 packed rows per lane, LPR = 32 -> 128 columns x 256 k.
// At M = 1, 8 packed rows per lane (128 columns x 512 k, half the splits) where the group
// size allows: 4.84 -> 4.55 us for config 0 (GPTQ sym 4096 x 4096) and 9.67 -> 8.87 us for
// GPTQ 4096 -> 14336 (graph replays); at M = 4 the deeper tile was slower (16.2 -> 17.0 us).
// At M = 2..4, 16 lanes per row where N and K allow (64 columns x 512 k, half the splits
// of the 128-column tile at the same workgroup count): M=4, 4096 -> 6144 9.1 -> 8.5 us; at
// M = 1 the 128-column tile is faster (4.56 vs 4.64 us for config 0).
constexpr int GQ_CW = 4, GQ_RL = 4, GQ_RL1 = 8, GQ_WAVES = 4, GQ_LPR = 32, GQ_LPRN = 16;
constexpr int gq_cols(int lpr) { return lpr * GQ_CW; }
constexpr int gq_rows(int lpr, int rl) { return (64 / lpr) * GQ_WAVES * rl * 8; }
constexpr int GQ_ROWS1 = gq_rows(GQ_LPR, GQ_RL1);
// AWQ, M = 2..8, matrix-core dot: CW = 2 words per lane (256 columns). Wide tile: R = 128
// rows per wave, 8 waves (1024 rows per workgroup: a quarter of the split-K partials of the
// narrow tile, which rereads M x N fp32 per split); narrow tile (R = 64, 4 waves, 256 rows)
// for K or group sizes the wide one does not divide. At K=4096 -> N=14336 / K=14336 ->
// N=4096 the wide tile takes M=2: 9.4 / 10.3 us, M=4: 11.4 / 11.9 us, M=8: 14.5 / 15.8 us
// against 10.6 / 12.1, 11.9 / 15.4, 17.7 / 24.6 us for the narrow one (4 waves x 128 rows:
// 15.3 / 19.0 us at M=8; 16 waves x 64 rows: 15.7 / 17.0 us).
constexpr int AM_CW = 2, AM_PF = 16;
constexpr int AM_R = 64, AM_WAVES = 4;
constexpr int AMW_R = 128, AMW_WAVES = 8;
constexpr int AM_COLS = 128 * AM_CW, AM_ROWS = AM_R * AM_WAVES, AMW_ROWS = AMW_R * AMW_WAVES;
// AWQ, M = 3..8, row-paired matrix-core kernel: 8 (or 4) waves x 128 rows per workgroup
constexpr int AR_MIN_M = 3, AR_WAVES = 8, AR_ROWS = 128 * AR_WAVES;
}  // namespace

GemvShape gemv_shape(int fmt, int M, int N, int K, int G, bool xcd_placement, bool bf16) {
    GemvShape s{};
    // AWQ: the row-paired matrix-core kernel for M = 3..8 where its tile fits (K a multiple of
    // 1024, groups of 128 rows or more); the block-diagonal matrix-core kernel for M = 2 and
    // for other shapes (M = 2: 10.3 vs 11.4 us, M = 4: 12.0 vs 14.5 us at K=4096, N=14336
    // against the VALU kernel), VALU dot2 at M = 1 (with the 512-row tile and the fixed-point
    // hand-off: 14336 -> 4096 8.40 vs 8.65 us, 8192 -> 4096 6.25 vs 7.70 us, 4096 -> 14336
    // 8.47 vs 9.20 us against the matrix-core kernel) and for shapes the matrix-core tile
    // rejects
    const bool mfma_fits = N % AM_COLS == 0 && K % AM_ROWS == 0 && G % AM_R == 0 && K % G == 0;
    const bool wide_fits = mfma_fits && K % AMW_ROWS == 0 && G % AMW_R == 0;
    const bool rows_fits = N % 256 == 0 && K % AR_ROWS == 0 && G % 128 == 0 && K % G == 0 &&
                           (size_t)K * N / 2 < ((size_t)1 << 31);
    if (fmt == FMT_AWQ && M >= AR_MIN_M && M <= GEMV_MFMA_MAX_M && rows_fits) {
        s.ok = true; s.mfma = true; s.awq_rows = true; s.col_tiles = N / 256;
        // 4 waves (512-row workgroups) where 8 would leave fewer than 64 workgroups (graph
        // replays, one GPU's share of an 8-way tensor-parallel layer, K=4096 -> N=1792: M=4
        // 7.7 -> 6.6 us, M=8 9.6 -> 8.6 us; 2 waves, 16 splits, 13.8 us at M=8)
        const int w = (N / 256) * (K / AR_ROWS) < 64 ? AR_WAVES / 2 : AR_WAVES;
        s.splits = K / (128 * w);
        s.threads = 64 * w;
    } else if (!bf16 && fmt == FMT_AWQ && M >= 2 && M <= GEMV_MFMA_MAX_M && mfma_fits) {
        s.ok = true; s.mfma = true; s.mfma_wide = wide_fits; s.col_tiles = N / AM_COLS;
        s.splits = K / (wide_fits ? AMW_ROWS : AM_ROWS);
        s.threads = 64 * (wide_fits ? AMW_WAVES : AM_WAVES);
    } else if (M >= 1 && M <= GEMV_MAX_M && fmt == FMT_AWQ) {
        if (N % 256 || K % AWQ_ROWS || G % AWQ_RL || K % G) return s;
        // weights are addressed through one buffer resource (32-bit offsets)
        if ((size_t)K * N / 2 >= ((size_t)1 << 31)) return s;
        s.awq_deep = M == 1 && K % AWQ_ROWS_DEEP == 0;
        // the 256-row tile where the 512-row one leaves fewer than 192 workgroups (4096 ->
        // 4096, 128 workgroups: 5.02 -> 4.33 us; 2048 -> 4096: 4.73 -> 3.74 us), the 512-row
        // tile from 192 up (4096 -> 6144: 5.44 vs 5.57 us; 4096 -> 8192: 6.01 vs 6.07 us)
        if (s.awq_deep && (N / 256) * (K / AWQ_ROWS_DEEP) < 192 && K / AWQ_ROWS <= FIX_MAX_SPLITS)
            s.awq_deep = false;
        s.ok = true; s.col_tiles = N / 256; s.splits = K / (s.awq_deep ? AWQ_ROWS_DEEP : AWQ_ROWS);
        s.threads = 64 * (s.awq_deep ? AWQ_WAVES_DEEP : AWQ_WAVES);
    } else if (M >= 1 && M <= GEMV_MAX_M) {
        if (G % (GQ_RL * 8) || K % G) return s;
        s.gptq_narrow = M > 1 && N % gq_cols(GQ_LPRN) == 0 && K % gq_rows(GQ_LPRN, GQ_RL) == 0;
        const int lpr = s.gptq_narrow ? GQ_LPRN : GQ_LPR, rows = gq_rows(lpr, GQ_RL);
        if (N % gq_cols(lpr) || K % rows) return s;
        s.gptq_deep = M == 1 && K % GQ_ROWS1 == 0 && G % (GQ_RL1 * 8) == 0;
        // With the fixed-point hand-off the 256-row tile wins where the 512-row one leaves
        // fewer than 512 workgroups (4096 -> 6144: 5.13 -> 4.70 us, 4096 -> 4096: 4.06 ->
        // 4.02 us) and loses above (4096 -> 14336, 896 workgroups: 8.45 -> 9.11 us).
        if (s.gptq_deep && (N / gq_cols(lpr)) * (K / GQ_ROWS1) < 512 && K / rows <= FIX_MAX_SPLITS)
            s.gptq_deep = false;
        s.ok = true; s.col_tiles = N / gq_cols(lpr); s.splits = K / (s.gptq_deep ? GQ_ROWS1 : rows);
        s.threads = 64 * GQ_WAVES;
    } else {
        return s;
    }
    // The XCD-local hand-off pays off at M = 1 (partials stay in L2: 9.8 vs 10.1 us for
    // K=4096, N=14336). With more rows the dirty partials the L2s write back at the end of
    // the kernel cost more than the shorter round trips save, so M > 1 keeps device scope.
    s.xcd = xcd_placement && M == 1 && s.splits > 1 && s.col_tiles % 8 == 0;
    return s;
}

template <int M, bool XCD, bool FIX, typename E>
static void launch_gemv_mx(int fmt, const GemvParams& p, const GemvShape& s, hipStream_t st) {
    const dim3 grid = XCD ? dim3(s.col_tiles * s.splits) : dim3(s.col_tiles, s.splits);
    const dim3 block(s.threads);
    constexpr bool H = std::is_same<E, half_t>::value;   // the block-diagonal GEMV is fp16 only
    if (fmt == FMT_AWQ && s.mfma) {
        if constexpr (M >= AR_MIN_M && M <= GEMV_MFMA_MAX_M && !XCD) {
            if (s.awq_rows) {
                if (s.threads == 64 * AR_WAVES)
                    hipLaunchKernelGGL((gemv_awq_rows_kernel<M, AR_WAVES, FIX, E>), grid, block, 0, st, p);
                else
                    hipLaunchKernelGGL((gemv_awq_rows_kernel<M, AR_WAVES / 2, FIX, E>), grid, block, 0, st, p);
                return;
            }
        }
        if constexpr (H && M <= GEMV_MFMA_MAX_M) {
            if (s.mfma_wide)
                hipLaunchKernelGGL((gemv_awq_mfma_kernel<M, AM_CW, AMW_R, AMW_WAVES, AM_PF, XCD, FIX>), grid, block, 0, st, p);
            else
                hipLaunchKernelGGL((gemv_awq_mfma_kernel<M, AM_CW, AM_R, AM_WAVES, AM_PF, XCD, FIX>), grid, block, 0, st, p);
        }
    } else if constexpr (M <= GEMV_MAX_M) {
        if constexpr (M == 1) {
            if (fmt != FMT_AWQ && s.gptq_deep) {
                if (fmt == FMT_GPTQ)
                    hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ, M, GQ_CW, GQ_RL1, GQ_WAVES, GQ_LPR, XCD, FIX, E>), grid, block, 0, st, p);
                else
                    hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ_SYM, M, GQ_CW, GQ_RL1, GQ_WAVES, GQ_LPR, XCD, FIX, E>), grid, block, 0, st, p);
                return;
            }
        }
        if constexpr (M > 1) {
            if (fmt != FMT_AWQ && s.gptq_narrow) {
                if (fmt == FMT_GPTQ)
                    hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ, M, GQ_CW, GQ_RL, GQ_WAVES, GQ_LPRN, XCD, FIX, E>), grid, block, 0, st, p);
                else
                    hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ_SYM, M, GQ_CW, GQ_RL, GQ_WAVES, GQ_LPRN, XCD, FIX, E>), grid, block, 0, st, p);
                return;
            }
        }
        if constexpr (M == 1) {
            if (fmt == FMT_AWQ && s.awq_deep) {
                hipLaunchKernelGGL((gemv_awq_kernel<M, AWQ_CW, AWQ_RL, AWQ_WAVES_DEEP, XCD, FIX, E>), grid, block, 0, st, p);
                return;
            }
        }
        if (fmt == FMT_AWQ)
            hipLaunchKernelGGL((gemv_awq_kernel<M, AWQ_CW, AWQ_RL, AWQ_WAVES, XCD, FIX, E>), grid, block, 0, st, p);
        else if (fmt == FMT_GPTQ)
            hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ, M, GQ_CW, GQ_RL, GQ_WAVES, GQ_LPR, XCD, FIX, E>), grid, block, 0, st, p);
        else
            hipLaunchKernelGGL((gemv_gptq_kernel<FMT_GPTQ_SYM, M, GQ_CW, GQ_RL, GQ_WAVES, GQ_LPR, XCD, FIX, E>), grid, block, 0, st, p);
    }
}

template <int M, typename E>
static hipError_t launch_gemv_m(int fmt, const GemvParams& p, const GemvShape& s, hipStream_t st) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (M > GEMV_MAX_M && !(fmt == FMT_AWQ && s.mfma)) return hipErrorInvalidValue;
    if (!std::is_same<E, half_t>::value && s.mfma && !s.awq_rows) return hipErrorInvalidValue;
    // the hand-off protocol is a template parameter: each kernel carries only the one it uses
    if (p.fixed) {
        if (s.xcd) launch_gemv_mx<M, true, true, E>(fmt, p, s, st);
        else launch_gemv_mx<M, false, true, E>(fmt, p, s, st);
    } else {
        if (s.xcd) launch_gemv_mx<M, true, false, E>(fmt, p, s, st);
        else launch_gemv_mx<M, false, false, E>(fmt, p, s, st);
    }
    return hipGetLastError();
}

hipError_t launch_gemv(int fmt, const GemvParams& p, const GemvShape& s, hipStream_t st, bool bf16) {
    if (bf16) {   // the VALU kernels and the row-paired AWQ kernel
        switch (p.M) {
            case 1: return launch_gemv_m<1, bf16_t>(fmt, p, s, st);
            case 2: return launch_gemv_m<2, bf16_t>(fmt, p, s, st);
            case 3: return launch_gemv_m<3, bf16_t>(fmt, p, s, st);
            case 4: return launch_gemv_m<4, bf16_t>(fmt, p, s, st);
            case 5: return launch_gemv_m<5, bf16_t>(fmt, p, s, st);
            case 6: return launch_gemv_m<6, bf16_t>(fmt, p, s, st);
            case 7: return launch_gemv_m<7, bf16_t>(fmt, p, s, st);
            case 8: return launch_gemv_m<8, bf16_t>(fmt, p, s, st);
            default: return hipErrorInvalidValue;
        }
    }
    switch (p.M) {
        case 1: return launch_gemv_m<1, half_t>(fmt, p, s, st);
        case 2: return launch_gemv_m<2, half_t>(fmt, p, s, st);
        case 3: return launch_gemv_m<3, half_t>(fmt, p, s, st);
        case 4: return launch_gemv_m<4, half_t>(fmt, p, s, st);
        case 5: return launch_gemv_m<5, half_t>(fmt, p, s, st);
        case 6: return launch_gemv_m<6, half_t>(fmt, p, s, st);
        case 7: return launch_gemv_m<7, half_t>(fmt, p, s, st);
        case 8: return launch_gemv_m<8, half_t>(fmt, p, s, st);
        default: return hipErrorInvalidValue;
    }
}

// Workgroup -> XCD placement probe: workgroup b records its XCC_ID.
__global__ void xcc_probe_kernel(uint32_t* out) {
    if (threadIdx.x == 0) {
        uint32_t x;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
        out[blockIdx.x] = x & 0xFu;
    }
}

hipError_t check_xcd_placement(bool* ok) {
    constexpr int B = 4096;
    *ok = false;
    uint32_t* d = nullptr;
    hipError_t e = hipMalloc(&d, B * sizeof(uint32_t));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(B), dim3(64), 0, 0, d);
    e = hipGetLastError();
    uint32_t h[B];
    if (e == hipSuccess) e = hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return e;
    bool same = true;
    for (int b = 8; b < B; ++b) same = same && h[b] == h[b % 8];
    *ok = same;
    return hipSuccess;
}

}  // namespace w4a16
