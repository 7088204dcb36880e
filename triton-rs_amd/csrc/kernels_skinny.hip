// Small-batch W4A16 GEMM (5 <= M <= 64) on MFMA: the weight stream is the cost (HBM-bound),
// so the kernel is built to keep loads in flight and to need few workgroup-to-workgroup
// reductions.
//
// A workgroup owns a strip of WN = 16*CPL columns; its waves (4, or 8 for GPTQ 32-row tiles
// and, where K allows, GPTQ 64-row tiles) split the strip's K range and stream independently
// (no LDS staging, no barrier in the main loop). Each lane keeps a ring of PF k32 steps of loads in flight: its packed words, the
// activation fragments and the group's scales/zeros. Every load of the steady state is
// unconditional (rows past M are loaded clamped and zeroed at use), so the compiler's
// wait counts let each step wait for its own slot only. Words are dequantised bit-exactly
// (W16 = RNE_f16((q - z) * s), crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:246-260,
// awq_gemm_int4_typed.rs:213-228) straight into MFMA B-operand registers and multiplied
// with v_mfma_f32_16x16x32_f16 (fp32 accumulation, the reference's tt.dot). The waves'
// accumulators are summed in LDS; when the strip count alone cannot fill the GPU the K
// range is also split across workgroups, joined by the counter hand-off of splitk.h.
//
// Operand layouts: slot j of MFMA c is output column
// n0 + CPL*j + c; GPTQ k-blocks are consumed in the unpack order (k0,k4)(k1,k5)(k2,k6)(k3,k7)
// with A permuted to match, AWQ in natural order via row pairs.
//
// Act-order (GIDX, GPTQ formats): the group of row k is g_idx[k] instead of k / G, so the
// scale and zero change from row to row. The workgroup first builds an LDS table holding,
// for every group and every column of its strip, the scale and the zero (as fp16 1024 + z)
// in one 32-bit entry; each k row then gathers its entries by g_idx[k]. The arithmetic per
// weight is unchanged, (fp16(1024 + q) - fp16(1024 + z)) * s, so the weights stay bit-exact.
// GIDX = 2 also stages the workgroup's slice of g_idx in LDS, as clamped table offsets (one
// load per thread instead of two 32-byte loads per lane and k32 step, which the 16 lanes of
// a k block all repeat, and no index arithmetic in the steps);
// GIDX = 1 (slice too large for the LDS budget) reads g_idx per step from global memory.
#include <type_traits>

#include "device_common.h"
#include "launch.h"
#include "splitk.h"

namespace w4a16 {

namespace {
// waves per workgroup: 8 for GPTQ 32-row tiles (the same wave count with half the workgroup
// splits, so half the split-K partials: config 2 M=32 12.3 -> 11.9 us plain, 15.3 -> 14.1 us
// act-order; at M=16 the 4-wave tile was faster, 9.7 vs 10.9 us); 4 otherwise (64-row tiles
// and AWQ, whose 8-column strips would not fit the reduction buffer twice: AWQ M=32
// 4096 -> 14336 22.2 us with 4 waves against 30.9 us with 8)
constexpr int skinny_waves(int fmt, int bm, int cpl) {
    return fmt != FMT_AWQ && bm == 32 && cpl < 8 ? 8 : 4;
}
__device__ __forceinline__ half2_t deq2(half2_t h, half2_t hz, half2_t hs) { return (h - hz) * hs; }
__device__ __forceinline__ half8_t cat8(half2_t a, half2_t b, half2_t c, half2_t d) {
    return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}
}  // namespace

// SPW: k32 steps per wave when known at compile time (SPW = PF: the prologue issues every
// step and no loop is emitted), 0 for the runtime count p.steps_per_wave.
// RG (plain group order): every ring round of PF steps lies in one group (G % (32 PF) == 0
// and steps_per_wave % PF == 0), so the round's first slot alone loads the scales and zeros,
// and the zero points and scales are splatted once per round instead of once per step.
// WV: waves per workgroup when it differs from skinny_waves (8 for 64-row GPTQ tiles, chosen
// on the host where K allows); 0 for the default.
// E: the element type of x, the scales and the output. With bf16 a weight is
// RNE_bf16((q - z) * s) (deq2_bf16: exact fp32 product, one rounding) and the MFMA is the
// bf16 one; the act-order table then holds (bf16 scale | z << 16).
template <int FMT, int BM, int CPL, int PF, int GIDX, bool XCD, int SPW, bool RG = false, int WV = 0,
          typename E = half_t>
__global__ void __launch_bounds__(64 * (WV ? WV : skinny_waves(FMT, BM, CPL))) skinny_kernel(SkinnyParams p) {
    constexpr bool BF = std::is_same<E, bf16_t>::value;
    typedef typename vec8<E>::type v8_t;
    static_assert(!RG || !GIDX, "one group per round needs plain group order");
    static_assert(!GIDX || FMT != FMT_AWQ, "act-order is a GPTQ layout");
    static_assert(CPL == 4 || (CPL == 2 && FMT != FMT_AWQ) || (CPL == 8 && FMT == FMT_AWQ),
                  "columns per lane");
    constexpr int W = WV ? WV : skinny_waves(FMT, BM, CPL), NT = 64 * W;
    // 64-row tiles of 8 waves reduce in two rounds through a 4-wave buffer (the single-round
    // buffer would take 133 KB of LDS)
    constexpr int RW = (BM == 64 && W == 8) ? 4 : W;
    static_assert(NT <= FINISH_MAX_THREADS, "split-K finish buffer");
    constexpr int RB = BM / 16;
    constexpr int WN = 16 * CPL;
    constexpr int WPS = (FMT == FMT_AWQ) ? 8 : CPL;   // packed words per lane per k32 step
    constexpr int SW = (CPL + 1) / 2;                  // scale words (2 halfs each) per lane

    __shared__ float red[RW][BM][WN + 1];
    __shared__ int flag;
    // GIDX: [groups][WN] of (scale | fp16(1024 + z) << 16) (bf16: scale | z << 16), then
    // (GIDX = 2) the g_idx of the
    // workgroup's W * spw * 32 rows
    extern __shared__ __attribute__((aligned(16))) uint32_t gtab[];   // 16-byte table accesses

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kb = lane >> 4;
    int ct, split;
    tile_of_block<XCD>(p.col_tiles, p.splits, ct, split);
    constexpr int SC = XCD ? SCOPE_XCD : SCOPE_DEVICE;
    const int n0 = ct * WN;
    const int nl = n0 + CPL * j;              // first output column of this lane
    const int NW = p.N >> 3;
    const int spw = SPW ? SPW : p.steps_per_wave;
    const int step0 = (split * W + wave) * spw;  // first k32 step of this wave

    // ------------------------------------------------ per-step loads into ring slot u
    uint32_t bw[PF][WPS];
    u32x4 areg[PF][RB];
    uint32_t sreg[PF][SW], zreg[PF];
    int32_t greg[PF][GIDX == 1 ? 8 : 1];
    int goff[PF];   // GIDX = 2: offset of the lane's 8 rows in the LDS g_idx slice

    auto issue = [&](int u, int step) {
        const int kg = 32 * step;
        // packed weights
        if constexpr (FMT == FMT_AWQ) {
            const int wcol = (CPL == 8) ? (n0 >> 3) + j : (nl >> 3);
            const uint32_t off0 = (uint32_t)(kg + 8 * kb) * (uint32_t)NW + (uint32_t)wcol;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                bw[u][r] = ld_stream(at_bytes(p.qweight, 4u * (off0 + (uint32_t)r * (uint32_t)NW)));
        } else {
            const uint32_t off = (uint32_t)((kg >> 3) + kb) * (uint32_t)p.N + (uint32_t)nl;
            if constexpr (CPL == 2) {
                const u32x2 v = ld_stream2(at_bytes(p.qweight, 4u * off));
                bw[u][0] = v.x; bw[u][1] = v.y;
            } else {
#pragma unroll
                for (int h = 0; h < CPL / 4; ++h) {
                    const u32x4 v = ld_stream4(at_bytes(p.qweight, 4u * (off + 4 * h)));
                    bw[u][4 * h + 0] = v.x; bw[u][4 * h + 1] = v.y;
                    bw[u][4 * h + 2] = v.z; bw[u][4 * h + 3] = v.w;
                }
            }
        }
        // activation fragments: row 16 r + j, k = kg + 8 kb .. + 7; rows >= M load row M - 1
        // and are zeroed where they are used, so that every lane issues every load
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int m = min(16 * r + j, p.M - 1);
            areg[u][r] = *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.K + kg + 8 * kb);
        }
        if constexpr (GIDX == 2) {
            goff[u] = (step - split * W * spw) * 32 + 8 * kb;
            return;
        } else if constexpr (GIDX == 1) {
            // groups of the lane's 8 k rows
            const u32x4* gp = reinterpret_cast<const u32x4*>(p.g_idx + kg + 8 * kb);
            const u32x4 g0 = gp[0], g1 = gp[1];
            greg[u][0] = g0.x; greg[u][1] = g0.y; greg[u][2] = g0.z; greg[u][3] = g0.w;
            greg[u][4] = g1.x; greg[u][5] = g1.y; greg[u][6] = g1.z; greg[u][7] = g1.w;
            return;
        }
        if constexpr (RG) {
            if (u != 0) return;   // the round's group comes with its first step
        }
        // scales and zero word of the lane's columns for this step's group
        const int g = kg / p.G;
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(p.scales + (size_t)g * p.N + nl);
        if constexpr (CPL == 8) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(sp);
            sreg[u][0] = v.x; sreg[u][1] = v.y; sreg[u][2] = v.z; sreg[u][3] = v.w;
        } else if constexpr (CPL == 4) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(sp);
            sreg[u][0] = v.x; sreg[u][1] = v.y;
        } else {
            sreg[u][0] = sp[0];
        }
        zreg[u] = (FMT == FMT_GPTQ_SYM) ? 0u : p.qzeros[(size_t)g * NW + (nl >> 3)];
    };

    float4_t acc[RB][CPL];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[r][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Act-order table: entry (g, c) = group g, strip column c at gtab[g * WN + c]. Thread work
    // comes in chunks of 8 columns of one group: one 16-byte load of their scales and one zero
    // word. Loads of one wave complete in issue order, so where the chunks fit TC per thread
    // they are loaded into registers before the weight stream and written to LDS after it has
    // been issued; the table is then ready about when the first weights arrive (loaded after
    // the stream, its build waited for all of it: config 2 M=16 12.5 -> 10.9 us). The g_idx
    // slice of GIDX = 2 is loaded the same way, 4 rows per load.
    const int ngroups = (p.K + p.G - 1) / p.G;
    constexpr int CPW = WN / 8;                       // chunks per group
    constexpr int TC = GIDX ? 2 : 1;
    constexpr int GC = GIDX == 2 ? 4 : 1;
    const int tab_chunks = GIDX ? ngroups * CPW : 0;
    const int tab_n = ngroups * WN;
    const bool tab_early = GIDX && tab_chunks <= TC * NT;
    const int gsl_rows = GIDX == 2 ? W * spw * 32 : 0;      // rows of the workgroup
    const int gsl_chunks = gsl_rows / 4;
    const bool gsl_early = GIDX == 2 && gsl_chunks <= GC * NT;
    const int32_t* gsrc = p.g_idx + (size_t)split * gsl_rows;
    uint32_t* gsl = gtab + tab_n;
    // the slice holds each row's table offset, clamp(g_idx, 0, groups - 1) * WN, so that the
    // steps read it without per-lane arithmetic
    auto gsl_entry = [&](u32x4 g) {
        const int hi = ngroups - 1;
        return u32x4{(uint32_t)(min(max((int)g.x, 0), hi) * WN), (uint32_t)(min(max((int)g.y, 0), hi) * WN),
                     (uint32_t)(min(max((int)g.z, 0), hi) * WN), (uint32_t)(min(max((int)g.w, 0), hi) * WN)};
    };
    u32x4 tsv[TC], gsv[GC];
    uint32_t tzv[TC];
    auto tab_load = [&](int c, u32x4& sv, uint32_t& zw) {
        const int g = c / CPW, b = c - g * CPW;
        sv = *reinterpret_cast<const u32x4*>(p.scales + (size_t)g * p.N + n0 + 8 * b);
        zw = (FMT == FMT_GPTQ_SYM) ? 0u : p.qzeros[(size_t)g * NW + (n0 >> 3) + b];
    };
    auto tab_store = [&](int c, const u32x4& sv, uint32_t zw) {
        const int g = c / CPW, b = c - g * CPW;
        uint32_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {   // column n0 + 8 b + i: nibble i of its zero word
            const int z = (FMT == FMT_GPTQ_SYM) ? 8 : nib(zw, i) + p.zero_offset;
            const uint32_t zf = BF ? (uint32_t)z : __builtin_bit_cast(uint16_t, (half_t)(1024 + z));
            const uint32_t sw = i < 2 ? sv.x : i < 4 ? sv.y : i < 6 ? sv.z : sv.w;
            e[i] = ((i & 1) ? (sw >> 16) : (sw & 0xFFFFu)) | (zf << 16);
        }
        uint32_t* dst = gtab + g * WN + 8 * b;
        reinterpret_cast<u32x4*>(dst)[0] = u32x4{e[0], e[1], e[2], e[3]};
        reinterpret_cast<u32x4*>(dst)[1] = u32x4{e[4], e[5], e[6], e[7]};
    };
    if constexpr (GIDX != 0) {
        if (tab_early) {
#pragma unroll
            for (int e = 0; e < TC; ++e)   // in range: loads unconditional
                tab_load(min((int)threadIdx.x + e * NT, tab_chunks - 1), tsv[e], tzv[e]);
        }
        if (gsl_early) {
#pragma unroll
            for (int e = 0; e < GC; ++e)
                gsv[e] = reinterpret_cast<const u32x4*>(gsrc)[min((int)threadIdx.x + e * NT, gsl_chunks - 1)];
        }
    }

    // prologue: PF steps in flight (a wave with fewer steps re-reads its last one, so the
    // number of loads in flight is known at compile time)
#pragma unroll
    for (int u = 0; u < PF; ++u) issue(u, step0 + min(u, spw - 1));

    if constexpr (GIDX != 0) {
        if (tab_early) {
#pragma unroll
            for (int e = 0; e < TC; ++e) {
                const int c = (int)threadIdx.x + e * NT;
                if (c < tab_chunks) tab_store(c, tsv[e], tzv[e]);
            }
        } else {
            for (int c = threadIdx.x; c < tab_chunks; c += NT) {
                u32x4 sv;
                uint32_t zw;
                tab_load(c, sv, zw);
                tab_store(c, sv, zw);
            }
        }
        if constexpr (GIDX == 2) {
            if (gsl_early) {
#pragma unroll
                for (int e = 0; e < GC; ++e) {
                    const int c = (int)threadIdx.x + e * NT;
                    if (c < gsl_chunks) reinterpret_cast<u32x4*>(gsl)[c] = gsl_entry(gsv[e]);
                }
            } else {
                for (int c = threadIdx.x; c < gsl_chunks; c += NT)
                    reinterpret_cast<u32x4*>(gsl)[c] = gsl_entry(reinterpret_cast<const u32x4*>(gsrc)[c]);
            }
        }
        __syncthreads();
    }

    // zero point (as fp16 1024 + z) and scale per column, splatted (bf16: the scale and
    // -z * s in fp32); with RG they are set by the first step of a round and kept for the
    // others
    half2_t hz[CPL], hs[CPL];
    float fs[CPL], fnz[CPL];
    // the element pair of the nibbles at bits 0 and 16 of v, dequantised for column c
    auto dq = [&](uint32_t v, int c) __attribute__((always_inline)) -> uint32_t {
        if constexpr (BF) return deq2_bf16(v, fs[c], fnz[c]);
        else return as_u32(deq2(nib_pair(v), hz[c], hs[c]));
    };

    // one k32 step from ring slot u
    auto compute = [&](int u) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < (GIDX != 0 || (RG && u != 0) ? 0 : CPL); ++c) {
            const int cw = (nl & 7) + c;   // column within its qzeros word
            int z;
            if constexpr (FMT == FMT_GPTQ_SYM) z = 8;
            else if constexpr (FMT == FMT_AWQ) z = nib(zreg[u], awq_slot(cw));
            else z = nib(zreg[u], cw) + p.zero_offset;
            if constexpr (BF) {
                const uint32_t sw = sreg[u][c >> 1];
                fs[c] = bf16_bits_to_f32((c & 1) ? sw >> 16 : sw & 0xFFFFu);
                fnz[c] = -(float)z * fs[c];
            } else {
                const half_t zh = (half_t)(1024 + z);
                hz[c] = half2_t{zh, zh};
                const half2_t sv = as_h2(sreg[u][c >> 1]);
                const half_t sc = (c & 1) ? sv.y : sv.x;
                hs[c] = half2_t{sc, sc};
            }
        }
        // dequantise B fragments
        v8_t bf[CPL];
        if constexpr (FMT == FMT_AWQ) {
            uint32_t pr[4][CPL];
#pragma unroll
            for (int rp = 0; rp < 4; ++rp) {
                const uint32_t a = bw[u][2 * rp], b = bw[u][2 * rp + 1];
                const uint32_t p0 = perm(b, a, 0x05040100u);   // slots 0-3 of both rows
                const uint32_t p1 = perm(b, a, 0x07060302u);   // slots 4-7
                if constexpr (CPL == 8) {
                    // the whole word: slot sl holds column awq_col_of_slot(sl)
#pragma unroll
                    for (int sl = 0; sl < 8; ++sl) {
                        const uint32_t src = sl < 4 ? p0 : p1;
                        const int col = awq_col_of_slot(sl);
                        pr[rp][col] = dq(src >> (4 * (sl & 3)), col);
                    }
                } else {
                    // columns 4h..4h+3 of the word: slots 2h, 4+2h, 2h+1, 5+2h
                    const int sh = 8 * (j & 1);
                    const uint32_t q0 = p0 >> sh, q1 = p1 >> sh;
                    pr[rp][0] = dq(q0, 0);
                    pr[rp][1] = dq(q1, 1);
                    pr[rp][2] = dq(q0 >> 4, 2);
                    pr[rp][3] = dq(q1 >> 4, 3);
                }
            }
#pragma unroll
            for (int c = 0; c < CPL; ++c) bf[c] = __builtin_bit_cast(v8_t, u32x4{pr[0][c], pr[1][c], pr[2][c], pr[3][c]});
        } else if constexpr (GIDX != 0) {
            // entries of rows k0..k7 for the lane's columns; a g_idx outside the table
            // is clamped into [0, groups - 1], as in the generic kernel
            int32_t gv[8];
            if constexpr (GIDX == 2) {
                const u32x4* gp = reinterpret_cast<const u32x4*>(gsl + goff[u]);
                const u32x4 g0 = gp[0], g1 = gp[1];
                gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w;
                gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) gv[i] = greg[u][i];
            }
            uint32_t t[8][CPL];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // GIDX = 2: the slice already holds the clamped group's table offset
                const uint32_t* row = gtab + CPL * j +
                    (GIDX == 2 ? (uint32_t)gv[i] : (uint32_t)min(max(gv[i], 0), ngroups - 1) * WN);
                if constexpr (CPL == 2) {
                    const u32x2 v = *reinterpret_cast<const u32x2*>(row);
                    t[i][0] = v.x; t[i][1] = v.y;
                } else {
#pragma unroll
                    for (int h = 0; h < CPL / 4; ++h) {
                        const u32x4 v = *reinterpret_cast<const u32x4*>(row + 4 * h);
                        t[i][4 * h + 0] = v.x; t[i][4 * h + 1] = v.y;
                        t[i][4 * h + 2] = v.z; t[i][4 * h + 3] = v.w;
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t w = bw[u][c];
                if constexpr (BF) {
                    // each half with its own row's scale and zero point, exact fp32 products
                    uint32_t pr[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t ea = t[q][c], eb = t[q + 4][c];
                        const float sa = bf16_bits_to_f32(ea & 0xFFFFu), sb = bf16_bits_to_f32(eb & 0xFFFFu);
                        const uint32_t x = (w >> (4 * q)) & 0x000F000Fu;
                        pr[q] = pack2(bf16_t{}, __builtin_fmaf((float)(x & 0xFFu), sa, -(float)(ea >> 16) * sa),
                                      __builtin_fmaf((float)(x >> 16), sb, -(float)(eb >> 16) * sb));
                    }
                    bf[c] = __builtin_bit_cast(v8_t, u32x4{pr[0], pr[1], pr[2], pr[3]});
                } else {
                    half2_t pr[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        // the pair holds rows k_q (low half) and k_{q+4} (high half)
                        const half2_t s2 = as_h2(perm(t[q + 4][c], t[q][c], 0x05040100u));
                        const half2_t z2 = as_h2(perm(t[q + 4][c], t[q][c], 0x07060302u));
                        pr[q] = deq2(nib_pair(w >> (4 * q)), z2, s2);
                    }
                    bf[c] = cat8(pr[0], pr[1], pr[2], pr[3]);
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t w = bw[u][c];
                bf[c] = __builtin_bit_cast(v8_t, u32x4{dq(w, c), dq(w >> 4, c), dq(w >> 8, c), dq(w >> 12, c)});
            }
        }
        // MFMAs
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            u32x4 a = areg[u][r];
            if (16 * r + j >= p.M) a = u32x4{0u, 0u, 0u, 0u};
            if constexpr (FMT != FMT_AWQ)   // k order (0,4)(1,5)(2,6)(3,7) as in the GPTQ unpack
                a = u32x4{perm(a.z, a.x, 0x05040100u), perm(a.z, a.x, 0x07060302u),
                          perm(a.w, a.y, 0x05040100u), perm(a.w, a.y, 0x07060302u)};
            const v8_t af = __builtin_bit_cast(v8_t, a);
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[r][c] = mfma16x16x32(af, bf[c], acc[r][c]);
        }
    };

    // Steady state: every step issues the step PF ahead, unconditionally, so the number of
    // loads in flight is the same on every iteration and each step waits only for its own
    // slot. The last 2 PF - 1 or fewer steps run in the tail.
    int s0 = 0;
    for (; s0 + 2 * PF <= spw; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            compute(u);
            issue(u, step0 + s0 + PF + u);
        }
    }
    const int rest = spw - s0 - PF;   // steps not yet issued (< PF; negative if spw < PF)
#pragma unroll
    for (int u = 0; u < PF; ++u) {
        if (s0 + u >= spw) break;
        compute(u);
        if (u < rest) issue(u, step0 + s0 + PF + u);
    }
#pragma unroll
    for (int u = 0; u < PF - 1; ++u)
        if (u < rest) compute(u);

    // ------------------------------------------------ reduce the W waves' K ranges
    if constexpr (RW < W) {
        // round 1: the upper waves hand their sums to the lower ones
        if (wave >= RW) {
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        red[wave - RW][16 * r + 4 * kb + i][CPL * j + c] = acc[r][c][i];
        }
        __syncthreads();
        if (wave < RW) {
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        acc[r][c][i] += red[wave][16 * r + 4 * kb + i][CPL * j + c];
        }
        __syncthreads();
    }
    if (wave < RW) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int c = 0; c < CPL; ++c) red[wave][16 * r + 4 * kb + i][CPL * j + c] = acc[r][c][i];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < BM * WN; o += NT) {
        const int m = o / WN, col = o - m * WN;
        if (m >= p.M) continue;
        float v = red[0][m][col];
#pragma unroll
        for (int w = 1; w < RW; ++w) v += red[w][m][col];
        const size_t off = (size_t)m * p.N + n0 + col;
        if (p.splits == 1) reinterpret_cast<E*>(p.out)[off] = (E)v;
        else st_partial<SC>(p.ws + (size_t)split * p.M * p.N + off, v);
    }
    if (p.splits == 1) return;
    if (splitk_arrive(splitk_counter(p.flags, ct), p.splits, &flag))
        splitk_finish_rows<SC, E>(p.ws, reinterpret_cast<E*>(p.out), p.splits, p.M, p.N, 0, p.M, n0, WN);
}

// ------------------------------------------------------------------ host side

SkinnyShape skinny_shape(int fmt, int M, int N, int K, int G, int num_cus, bool gidx,
                         bool xcd_placement) {
    SkinnyShape s{};
    if (M < 1 || M > 64 || K % 128) return s;
    // without g_idx a k32 step lies in one group; with it the group comes from the table
    if (gidx ? (fmt == FMT_AWQ || G < 1) : (G % 32 || K % G)) return s;
    s.bm = M <= 16 ? 16 : M <= 32 ? 32 : 64;
    const bool awq = fmt == FMT_AWQ;
    // GPTQ: 4 columns per lane where N allows (the wider strip re-reads the activations from
    // L2 half as often as 2). AWQ: a whole AWQ word (8 columns) per lane where N >= 4096 (with
    // 4, two lanes load each word: 4096 -> 14336 at M=16 21.4 -> 15.5 us, M=64 43.8 -> 32.0
    // us; at N=2048 the halved strip count cost more than it saved, 10.8 -> 12.4 us), else
    // half a word. (The 64-row, 8-column reduction buffer takes 132 KB of LDS: no room for
    // an act-order table, which AWQ never has.)
    auto pick_cpl = [&](int bm) {
        for (int c : {8, 4, 2}) {
            if (awq ? c < 4 : c > 4) continue;
            if (c == 8 && N < 4096) continue;   // small N: keep the strips
            if (N % (16 * c) == 0) return c;
        }
        return 0;
    };
    int cpl = pick_cpl(s.bm);
    // the 8-wave tile consumes K in steps of 256 rows; other K take the 64-row tile
    if (cpl && skinny_waves(fmt, s.bm, cpl) == 8 && K % 256) {
        s.bm = 64;
        cpl = pick_cpl(s.bm);
    }
    if (!cpl) return s;
    if (gidx) {
        s.lds = (size_t)((K + G - 1) / G) * 16 * cpl * sizeof(uint32_t);
        if (s.lds > SKINNY_GIDX_MAX_LDS) return s;
    }
    s.cpl = cpl;
    s.col_tiles = N / (16 * cpl);
    // split K across workgroups until ~2 workgroups per CU, keeping the fp32 partials
    // (splits * M * N * 4 bytes) under a quarter of the packed weights (K * N / 2 bytes) and
    // workgroups x M near 12K (measured optimum at K=4096, N=6144: 8 splits at M=16, 4 at
    // M=32, 2 at M=64; more splits cost more in partial traffic than they gain in width)
    // (counted in units of 4 waves: quads = splits x waves / 4)
    // AWQ with 8-column strips: up to 2 workgroups per CU at M <= 16, 1 above (measured at
    // M = 9..32 on both config-1 shapes: e.g. M=24, 4096 -> 14336 21.1 us with 224
    // workgroups against 26.6 with 448; M=32, 14336 -> 4096 21.5 with 256 against 32.3 with
    // 128)
    auto more = [&](int q) {
        if (cpl == 8) return (long long)s.col_tiles * 2 * q <= (M <= 16 ? 2 : 1) * num_cus;
        return (long long)s.col_tiles * 2 * q * M <= 12288;
    };
    int quads = 1;
    while (s.col_tiles * quads < 2 * num_cus && K % (128 * 2 * quads) == 0 &&
           2 * quads * 32 * M <= K && more(quads))
        quads *= 2;
    const int wq = skinny_waves(fmt, s.bm, cpl) / 4;
    int splits = quads >= wq ? quads / wq : 1;
    s.waves = skinny_waves(fmt, s.bm, cpl);
    // 64-row GPTQ tiles: 8 waves over the same workgroups (two waves per SIMD instead of one,
    // each with half the K range) where K divides
    if (s.bm == 64 && !awq && cpl < 8 && K % (256 * quads) == 0) {
        s.waves = 8;
        splits = quads;
    }
    s.splits = splits;
    s.steps_per_wave = K / (32 * s.waves * splits);
    // act-order: the workgroup's g_idx slice joins the table in LDS where the budget allows
    if (gidx && s.lds + (size_t)(K / splits) * sizeof(int32_t) <= SKINNY_GIDX_MAX_LDS) {
        s.gidx_lds = true;
        s.lds += (size_t)(K / splits) * sizeof(int32_t);
    }
    s.xcd = xcd_placement && splits > 1 && s.col_tiles % 8 == 0;
    s.ok = true;
    return s;
}

template <int FMT, int BM, int CPL, bool XCD, int WV, typename E>
static hipError_t launch_xw(const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    // 8-wave 64-row tiles keep a 2-step ring: two waves per SIMD need <= 256 registers
    constexpr int PF = FMT == FMT_AWQ ? 3 : WV == 8 ? 2 : 4;
    constexpr int NTH = 64 * (WV ? WV : skinny_waves(FMT, BM, CPL));
    const dim3 grid = XCD ? dim3(s.col_tiles * s.splits) : dim3(s.col_tiles, s.splits);
    if constexpr (FMT != FMT_AWQ) {
        if (p.g_idx) {
            // act-order waves with exactly one ring of steps run without a loop: the loop's
            // ring copies raise the kernel to 186 VGPRs, two waves per SIMD instead of three
            // (config 2 M=16: 14.3 -> 10.5 us)
            auto go = [&](auto kern) -> hipError_t {
                // static reduction buffer plus the group table may exceed the default 64 KiB
                const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)SKINNY_GIDX_MAX_LDS);
                if (attr != hipSuccess) return attr;
                hipLaunchKernelGGL(kern, grid, dim3(NTH), s.lds, st, p);
                return hipGetLastError();
            };
            if (s.gidx_lds) {
                if (s.steps_per_wave == PF) return go(&skinny_kernel<FMT, BM, CPL, PF, 2, XCD, PF, false, WV, E>);
                return go(&skinny_kernel<FMT, BM, CPL, PF, 2, XCD, 0, false, WV, E>);
            }
            if (s.steps_per_wave == PF) return go(&skinny_kernel<FMT, BM, CPL, PF, 1, XCD, PF, false, WV, E>);
            return go(&skinny_kernel<FMT, BM, CPL, PF, 1, XCD, 0, false, WV, E>);
        }
    }
    if constexpr (FMT != FMT_AWQ) {
        // one group per ring round (RG): the wave's rounds start on multiples of 32 PF rows
        const bool rg = p.G % (32 * PF) == 0 && s.steps_per_wave % PF == 0;
        if (s.steps_per_wave == PF) {   // as above: M=16, 4096 -> 6144 9.4 -> 8.6 us
            if (rg) hipLaunchKernelGGL((skinny_kernel<FMT, BM, CPL, PF, 0, XCD, PF, true, WV, E>), grid, dim3(NTH), 0, st, p);
            else hipLaunchKernelGGL((skinny_kernel<FMT, BM, CPL, PF, 0, XCD, PF, false, WV, E>), grid, dim3(NTH), 0, st, p);
            return hipGetLastError();
        }
        if (rg) {
            hipLaunchKernelGGL((skinny_kernel<FMT, BM, CPL, PF, 0, XCD, 0, true, WV, E>), grid, dim3(NTH), 0, st, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((skinny_kernel<FMT, BM, CPL, PF, 0, XCD, 0, false, WV, E>), grid, dim3(NTH), 0, st, p);
    return hipGetLastError();
}

template <int FMT, int BM, int CPL, bool XCD, typename E>
static hipError_t launch_x(const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    if constexpr (BM == 64 && FMT != FMT_AWQ && CPL < 8) {
        if (s.waves == 8) return launch_xw<FMT, BM, CPL, XCD, 8, E>(p, s, st);
    }
    return launch_xw<FMT, BM, CPL, XCD, 0, E>(p, s, st);
}

template <int FMT, int BM, int CPL, typename E>
static hipError_t launch_t(const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    return s.xcd ? launch_x<FMT, BM, CPL, true, E>(p, s, st) : launch_x<FMT, BM, CPL, false, E>(p, s, st);
}

template <int FMT, int BM, typename E>
static hipError_t launch_bm(const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    if constexpr (FMT != FMT_AWQ) {
        if (s.cpl == 2) return launch_t<FMT, BM, 2, E>(p, s, st);
    } else {
        if (s.cpl == 8) return launch_t<FMT, BM, 8, E>(p, s, st);
    }
    return launch_t<FMT, BM, 4, E>(p, s, st);
}

template <int FMT, typename E>
static hipError_t launch_fmt(const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    switch (s.bm) {
        case 16: return launch_bm<FMT, 16, E>(p, s, st);
        case 32: return launch_bm<FMT, 32, E>(p, s, st);
        default: return launch_bm<FMT, 64, E>(p, s, st);
    }
}

template <typename E>
static hipError_t launch_e(int fmt, const SkinnyParams& p, const SkinnyShape& s, hipStream_t st) {
    if (fmt == FMT_AWQ) return launch_fmt<FMT_AWQ, E>(p, s, st);
    if (fmt == FMT_GPTQ) return launch_fmt<FMT_GPTQ, E>(p, s, st);
    return launch_fmt<FMT_GPTQ_SYM, E>(p, s, st);
}

hipError_t launch_skinny(int fmt, const SkinnyParams& p, const SkinnyShape& s, hipStream_t st, bool bf16) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    return bf16 ? launch_e<bf16_t>(fmt, p, s, st) : launch_e<half_t>(fmt, p, s, st);
}

}  // namespace w4a16
