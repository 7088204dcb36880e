// MFMA W4A16 GEMM for M >= 5: small-batch decode (split over K) and prefill.
//
// C[m, n] = sum_k x[m, k] * W16[k, n], W16 = RNE_f16((q - z) * s) exactly as the reference
// dequantises (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:246-260,
// awq_gemm_int4_typed.rs:213-228), f16 x f16 products accumulated in fp32 by
// v_mfma_f32_16x16x32_f16 (the reference's tt.dot, :265 / :233), fp16 output.
//
// Workgroup = 4 waves side by side along N; each wave owns WN = 16*CPL columns and all BM
// rows of the tile, so every packed weight is loaded and dequantised exactly once per
// workgroup and never goes through LDS: a lane turns its packed words straight into its
// MFMA B-operand registers. The activation tile (BM x 128 k) is staged in LDS, double
// buffered, and shared by the four waves.
//
// MFMA 16x16x32 f16 operand layout (gfx950): lane l supplies A[l%16][8*(l/16) + i] and
// B[8*(l/16) + i][l%16] (i = 0..7) and receives D[4*(l/16) + r][l%16] (r = 0..3). The 16
// B columns of one MFMA need not be adjacent: slot j of MFMA c maps to output column
// CPL*j + c of the wave, so one lane's 128-bit load (GPTQ) or word (AWQ) covers CPL
// MFMAs. Within a k-block of 8 the order of k only has to agree between A and B:
//   GPTQ  a word holds 8 consecutive k of one column; unpacked as (k0,k4)(k1,k5)(k2,k6)(k3,k7)
//         and A is staged in that same order,
//   AWQ   a lane reads its word column from 8 consecutive rows and pairs rows (k, k+1) with
//         v_perm_b32, so k stays in natural order.
#include "device_common.h"
#include "launch.h"
#include "splitk.h"

namespace w4a16 {

namespace {
constexpr int SK = 128;        // k per A stage
constexpr int LDA = SK + 8;    // halfs per LDS row of A (272-byte rows)
// fp16 (q - z) * s for a pair built by nib_pair (1024 + q): exact subtract, one RNE multiply
__device__ __forceinline__ half2_t deq2(half2_t h, half2_t hz, half2_t hs) { return (h - hz) * hs; }

__device__ __forceinline__ half8_t cat8(half2_t a, half2_t b, half2_t c, half2_t d) {
    return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}
}  // namespace

// Words per lane per k32 step: GPTQ CPL columns x 8 k = CPL words; AWQ 8 rows x 1 word
// (CPL = 8) or 8 rows x half a word (CPL = 4).
template <int FMT, int CPL>
struct BTraits {
    static constexpr int WPS = (FMT == FMT_AWQ) ? 8 : CPL;
};

template <int FMT, int BM, int CPL>
__global__ void __launch_bounds__(256) mfma_gemm_kernel(MfmaParams p) {
    constexpr int RB = BM / 16;
    constexpr int WN = 16 * CPL;
    constexpr int WGN = 4 * WN;
    constexpr int WPS = BTraits<FMT, CPL>::WPS;
    constexpr int ACH = BM * (SK / 8) / 256;   // 16-byte A chunks per thread per stage
    static_assert(ACH >= 1, "BM too small");

    __shared__ __attribute__((aligned(16))) half_t As[2][BM][LDA];
    __shared__ int flag;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kb = lane >> 4;
    const int ct = blockIdx.x, mt = blockIdx.y, split = blockIdx.z;
    const int n_wave = ct * WGN + wave * WN;
    const int nl = n_wave + CPL * j;              // first output column of this lane
    const int m0 = mt * BM;
    const int k_begin = split * p.k_per_split;
    const int nstages = p.k_per_split / SK;
    const int NW = p.N >> 3;

    // ------------------------------------------------ global -> register loaders
    auto load_a = [&](int kst, u32x4 (&areg)[ACH]) {
#pragma unroll
        for (int q = 0; q < ACH; ++q) {
            const int idx = threadIdx.x + 256 * q;
            const int row = idx >> 4, cc = idx & 15;
            const int m = m0 + row;
            if (m < p.M)
                areg[q] = *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.K + kst + 8 * cc);
            else
                areg[q] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_a = [&](int buf, const u32x4 (&areg)[ACH]) {
#pragma unroll
        for (int q = 0; q < ACH; ++q) {
            const int idx = threadIdx.x + 256 * q;
            const int row = idx >> 4, cc = idx & 15;
            u32x4 v = areg[q];
            if constexpr (FMT != FMT_AWQ) {
                // (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> (x0,x4)(x1,x5)(x2,x6)(x3,x7)
                v = u32x4{perm(areg[q].z, areg[q].x, 0x05040100u), perm(areg[q].z, areg[q].x, 0x07060302u),
                          perm(areg[q].w, areg[q].y, 0x05040100u), perm(areg[q].w, areg[q].y, 0x07060302u)};
            }
            *reinterpret_cast<u32x4*>(&As[buf][row][8 * cc]) = v;
        }
    };
    // packed words of the 4 k32 steps of a stage
    auto load_b = [&](int kst, uint32_t (&bw)[4][WPS]) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int kg = kst + 32 * ks;
            if constexpr (FMT == FMT_AWQ) {
                const int wcol = (CPL == 8) ? (n_wave >> 3) + j : (nl >> 3);
                const uint32_t* src = p.qweight + (size_t)(kg + 8 * kb) * NW + wcol;
#pragma unroll
                for (int r = 0; r < 8; ++r) bw[ks][r] = ld_stream(src + (size_t)r * NW);
            } else {
                const uint32_t* src = p.qweight + (size_t)((kg >> 3) + kb) * p.N + nl;
#pragma unroll
                for (int h = 0; h < CPL / 4; ++h) {
                    const u32x4 v = ld_stream4(src + 4 * h);
                    bw[ks][4 * h + 0] = v.x; bw[ks][4 * h + 1] = v.y;
                    bw[ks][4 * h + 2] = v.z; bw[ks][4 * h + 3] = v.w;
                }
            }
        }
    };
    // scales (CPL halfs) and the zero word of the lane's columns, per k32 step
    auto load_sz = [&](int kst, uint32_t (&sreg)[4][CPL / 2], uint32_t (&zreg)[4]) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int g = (kst + 32 * ks) / p.G;
            const uint32_t* sp = reinterpret_cast<const uint32_t*>(p.scales + (size_t)g * p.N + nl);
            if constexpr (CPL == 8) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(sp);
                sreg[ks][0] = v.x; sreg[ks][1] = v.y; sreg[ks][2] = v.z; sreg[ks][3] = v.w;
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2*>(sp);
                sreg[ks][0] = v.x; sreg[ks][1] = v.y;
            }
            zreg[ks] = (FMT == FMT_GPTQ_SYM) ? 0u : p.qzeros[(size_t)g * NW + (nl >> 3)];
        }
    };

    float4_t acc[RB][CPL];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[r][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    u32x4 areg[ACH];
    uint32_t bw[4][WPS], bwn[4][WPS];
    uint32_t sreg[4][CPL / 2], zreg[4], sregn[4][CPL / 2], zregn[4];
    half2_t hz[CPL], hs[CPL];

    load_a(k_begin, areg);
    load_b(k_begin, bw);
    load_sz(k_begin, sreg, zreg);
    store_a(0, areg);
    __syncthreads();

    for (int s = 0; s < nstages; ++s) {
        const int kst = k_begin + s * SK;
        const bool more = s + 1 < nstages;
        if (more) {
            load_a(kst + SK, areg);
            load_b(kst + SK, bwn);
            load_sz(kst + SK, sregn, zregn);
        }
        const int buf = s & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int kg = kst + 32 * ks;
            if (ks == 0 || (kg % p.G) == 0) {
                // new group: per-column zero (as fp16 1024 + z) and scale, splatted
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int cw = (nl & 7) + c;  // column within its qzeros word
                    int z;
                    if constexpr (FMT == FMT_GPTQ_SYM) z = 8;
                    else if constexpr (FMT == FMT_AWQ) z = nib(zreg[ks], awq_slot(cw));
                    else z = nib(zreg[ks], cw) + p.zero_offset;
                    const half_t zh = (half_t)(1024 + z);
                    hz[c] = half2_t{zh, zh};
                    const half2_t sv = as_h2(sreg[ks][c >> 1]);
                    const half_t sc = (c & 1) ? sv.y : sv.x;
                    hs[c] = half2_t{sc, sc};
                }
            }
            // ---- dequantise this lane's B fragments
            half8_t bf[CPL];
            if constexpr (FMT == FMT_AWQ) {
                half2_t pr[4][CPL];   // [row pair][column]
#pragma unroll
                for (int rp = 0; rp < 4; ++rp) {
                    const uint32_t a = bw[ks][2 * rp], b = bw[ks][2 * rp + 1];
                    const uint32_t p0 = perm(b, a, 0x05040100u);   // slots 0-3 of both rows
                    const uint32_t p1 = perm(b, a, 0x07060302u);   // slots 4-7
                    if constexpr (CPL == 8) {
#pragma unroll
                        for (int sl = 0; sl < 8; ++sl) {
                            const uint32_t src = sl < 4 ? p0 : p1;
                            const int col = awq_col_of_slot(sl);
                            pr[rp][col] = deq2(nib_pair(src >> (4 * (sl & 3))), hz[col], hs[col]);
                        }
                    } else {
                        // columns 4h..4h+3 of the word: slots 2h, 4+2h, 2h+1, 5+2h
                        const int sh = 8 * (j & 1);
                        const uint32_t q0 = p0 >> sh, q1 = p1 >> sh;
                        pr[rp][0] = deq2(nib_pair(q0), hz[0], hs[0]);
                        pr[rp][1] = deq2(nib_pair(q1), hz[1], hs[1]);
                        pr[rp][2] = deq2(nib_pair(q0 >> 4), hz[2], hs[2]);
                        pr[rp][3] = deq2(nib_pair(q1 >> 4), hz[3], hs[3]);
                    }
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) bf[c] = cat8(pr[0][c], pr[1][c], pr[2][c], pr[3][c]);
            } else {
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const uint32_t w = bw[ks][c];
                    bf[c] = cat8(deq2(nib_pair(w), hz[c], hs[c]), deq2(nib_pair(w >> 4), hz[c], hs[c]),
                                 deq2(nib_pair(w >> 8), hz[c], hs[c]), deq2(nib_pair(w >> 12), hz[c], hs[c]));
                }
            }
            // ---- MFMAs: every row block against every column of the lane
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const half8_t af = *reinterpret_cast<const half8_t*>(&As[buf][16 * r + j][32 * ks + 8 * kb]);
#pragma unroll
                for (int c = 0; c < CPL; ++c)
                    acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[c], acc[r][c], 0, 0, 0);
            }
        }
        if (more) {
            store_a(buf ^ 1, areg);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int w = 0; w < WPS; ++w) bw[ks][w] = bwn[ks][w];
#pragma unroll
                for (int w = 0; w < CPL / 2; ++w) sreg[ks][w] = sregn[ks][w];
                zreg[ks] = zregn[ks];
            }
        }
        __syncthreads();
    }

    // ------------------------------------------------ epilogue
    if (p.splits == 1) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + 16 * r + 4 * kb + i;
                if (m >= p.M) continue;
                half_t v[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) v[c] = (half_t)acc[r][c][i];
                half_t* dst = p.out + (size_t)m * p.N + nl;
                if constexpr (CPL == 8)
                    *reinterpret_cast<half8_t*>(dst) = half8_t{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
                else
                    *reinterpret_cast<u32x2*>(dst) = u32x2{as_u32(half2_t{v[0], v[1]}), as_u32(half2_t{v[2], v[3]})};
            }
        return;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 16 * r + 4 * kb + i;
            if (m >= p.M) continue;
            float* dst = p.ws + (size_t)split * p.M * p.N + (size_t)m * p.N + nl;
#pragma unroll
            for (int c = 0; c < CPL; ++c) st_coherent(dst + c, acc[r][c][i]);
        }
    const int tile = mt * gridDim.x + ct;
    uint32_t* flags = p.counters + (size_t)tile * p.splits;
    if (splitk_arrive(flags, split, p.splits, &flag)) {
        const int rows = min(BM, p.M - m0);
        splitk_finish_rows(p.ws, p.out, flags, p.splits, p.M, p.N, m0, rows, ct * WGN, WGN);
    }
}

// ------------------------------------------------------------------ host side

MfmaShape mfma_shape(int fmt, int M, int N, int K, int G, int num_cus) {
    MfmaShape s{};
    if (M < 1 || K % SK || G % 32 || K % G) return s;
    s.bm = M <= 16 ? 16 : M <= 32 ? 32 : M <= 64 ? 64 : 128;
    // widest column tile that divides N; prefill prefers 4-column lanes (fewer accumulators)
    const int want = s.bm >= 128 ? 4 : 8;
    s.cpl = 0;
    for (int c = want; c >= 4; c /= 2)
        if (N % (64 * c) == 0) { s.cpl = c; break; }
    if (!s.cpl && N % 256 == 0) s.cpl = 4;
    if (!s.cpl) return s;
    s.col_tiles = N / (64 * s.cpl);
    s.row_tiles = (M + s.bm - 1) / s.bm;
    // split K until the grid has ~3 workgroups per CU (weights are then streamed by enough
    // waves); each split keeps a whole number of 128-k stages
    const int stages = K / SK;
    int splits = 1;
    while (s.col_tiles * s.row_tiles * splits < 3 * num_cus && stages % (2 * splits) == 0 &&
           splits < 64)
        splits *= 2;
    s.splits = splits;
    s.k_per_split = K / splits;
    s.ok = true;
    return s;
}

template <int FMT, int BM, int CPL>
static void launch_t(const MfmaParams& p, const MfmaShape& s, hipStream_t st) {
    hipLaunchKernelGGL((mfma_gemm_kernel<FMT, BM, CPL>), dim3(s.col_tiles, s.row_tiles, s.splits),
                       dim3(256), 0, st, p);
}

template <int FMT, int BM>
static void launch_bm(const MfmaParams& p, const MfmaShape& s, hipStream_t st) {
    if (s.cpl == 8) launch_t<FMT, BM, 8>(p, s, st);
    else launch_t<FMT, BM, 4>(p, s, st);
}

template <int FMT>
static void launch_fmt(const MfmaParams& p, const MfmaShape& s, hipStream_t st) {
    switch (s.bm) {
        case 16: launch_bm<FMT, 16>(p, s, st); break;
        case 32: launch_bm<FMT, 32>(p, s, st); break;
        case 64: launch_bm<FMT, 64>(p, s, st); break;
        default: launch_bm<FMT, 128>(p, s, st); break;
    }
}

hipError_t launch_mfma(int fmt, const MfmaParams& p, const MfmaShape& s, hipStream_t st) {
    (void)hipGetLastError();  // launch errors below are ours, not an earlier call's
    if (fmt == FMT_AWQ) launch_fmt<FMT_AWQ>(p, s, st);
    else if (fmt == FMT_GPTQ) launch_fmt<FMT_GPTQ>(p, s, st);
    else launch_fmt<FMT_GPTQ_SYM>(p, s, st);
    return hipGetLastError();
}

}  // namespace w4a16
