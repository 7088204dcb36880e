// Generic strided W4A16 GEMM: the reference kernels' full parameter list (any strides,
// any M/N/K, masked tails), with the dequantised tile staged in LDS and fed to
// v_mfma_f32_16x16x32_f16 (E = half_t) or v_mfma_f32_16x16x32_bf16 (E = bf16_t: activations,
// scales and output in bfloat16, W = RNE_bf16((q - z) * s); the reference kernels are generic
// over the element type, w4a16_gptq_gemm_typed.rs:65-67).
//
// Semantics follow crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:130-273 and
// awq_gemm_int4_typed.rs:116-241: W16 = RNE_f16((q - z) * s) element by element (bit-exact
// with the reference), f16 x f16 products accumulated in fp32, fp16 store. Two
// generalisations: the group of row k is g_idx[k] when g_idx is given (act-order), and the
// group is computed per row, so BK <= group_size is not required. Out-of-range A and W
// elements are read as 0 (the reference's masked loads leave them undefined).
#pragma once
#include "device_common.h"
#include "launch.h"

namespace w4a16 {

constexpr int STR_BM = 64, STR_BN = 64, STR_BK = 32;
constexpr int STR_LDA = STR_BK + 8;  // halfs per LDS row (pad: 80-byte rows)

template <int FMT, typename E = half_t>
__device__ __forceinline__ void strided_gemm_body(const StridedParams& p) {
    if (p.gate && *p.gate != p.gate_want) return;   // uniform: the whole grid returns
    typedef typename vec8<E>::type e8_t;
    __shared__ __attribute__((aligned(16))) E As[STR_BM][STR_LDA];
    __shared__ __attribute__((aligned(16))) E Bs[STR_BN][STR_LDA];   // [n][k]
    const E* pa = reinterpret_cast<const E*>(p.a);
    const E* ps = reinterpret_cast<const E*>(p.scales);
    E* pc = reinterpret_cast<E*>(p.c);

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // Tiles numbered m first: a grid of (ceil(m/64), ceil(n/64)) gives each workgroup the tile
    // (blockIdx.x, blockIdx.y); a smaller grid walks the rest in strides of its size.
    // The first barrier of every k step keeps a tile's LDS writes behind the previous tile's
    // MFMA reads.
    const int64_t tiles_m = (p.m + STR_BM - 1) / STR_BM, tiles = tiles_m * ((p.n + STR_BN - 1) / STR_BN);
    for (int64_t tile = blockIdx.x + (int64_t)blockIdx.y * gridDim.x; tile < tiles;
         tile += (int64_t)gridDim.x * gridDim.y) {
        const int m0 = (int)(tile % tiles_m) * STR_BM, n0 = (int)(tile / tiles_m) * STR_BN;

        float4_t acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

        // A loader: row t/4, k offset (t%4)*8.  B producer: column t%64, k offset (t/64)*8.
        const int a_row = t >> 2, a_k = (t & 3) * 8;
        const int b_col = t & 63, b_k = (t >> 6) * 8;
        const int gm = m0 + a_row, gn = n0 + b_col;

        for (int kb = 0; kb < p.k; kb += STR_BK) {
            // ---- A tile
            E av[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int kk = kb + a_k + i;
                av[i] = (gm < p.m && kk < p.k)
                            ? pa[(int64_t)gm * p.stride_am + (int64_t)kk * p.stride_ak]
                            : (E)0.f;
            }
            // ---- B tile: dequantise 8 consecutive k of column gn
            E bv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int kk = kb + b_k + i;
                E v = (E)0.f;
                if (gn < p.n && kk < p.k) {
                    uint32_t word;
                    int slot;
                    if constexpr (FMT == FMT_PREP) {
                        // prepared layout: strip gn / 16 is stride_qwk words, its table the first
                        // stride_qwn of them (rows of 16 entries, R per 128-row block)
                        const uint32_t* strip = p.qweight + (int64_t)(gn >> 4) * p.stride_qwk;
                        const int kb = kk >> 7, col = gn & 15;
                        word = strip[p.stride_qwn + kb * 256 + (col + 16 * ((kk >> 5) & 3)) * 4 + ((kk >> 3) & 3)];
                        const int R = p.group_size < 128 ? 128 / p.group_size : 1;
                        const int r = p.group_size < 128 ? (kk & 127) / p.group_size : 0;
                        // act-order (rows in the checkpoint's order): group g's entry is table
                        // row g (G / 128) for G >= 128, row g for G = 32, 64
                        const int ga = p.g_idx ? min(max(p.g_idx[kk], 0), (p.k - 1) / p.group_size) : 0;
                        const int trow = p.g_idx ? ga * (p.group_size >= 128 ? p.group_size / 128 : 1)
                                                 : kb * R + r;
                        const uint32_t e = strip[trow * 16 + col];
                        const E s = (E)(float)__builtin_bit_cast(half_t, (uint16_t)e);
                        v = dequant1(nib(word, prep_slot(kk & 7)), (int)(e >> 16), s);
                        bv[i] = v;
                        continue;
                    }
                    if constexpr (FMT == FMT_AWQ) {
                        word = p.qweight[(int64_t)kk * p.stride_qwk + (int64_t)(gn >> 3) * p.stride_qwn];
                        slot = awq_slot(gn);
                    } else {
                        word = p.qweight[(int64_t)(kk >> 3) * p.stride_qwk + (int64_t)gn * p.stride_qwn];
                        slot = kk & 7;
                    }
                    // act-order group, clamped into the scale table so a bad g_idx cannot
                    // read out of bounds
                    const int g = p.g_idx ? min(max(p.g_idx[kk], 0), (p.k - 1) / p.group_size)
                                          : kk / p.group_size;
                    uint32_t qz = 0;
                    if constexpr (FMT != FMT_GPTQ_SYM)
                        qz = p.qzeros[(int64_t)g * p.stride_qzk + (int64_t)(gn >> 3) * p.stride_qzn];
                    const E s = ps[(int64_t)g * p.stride_sk + (int64_t)gn * p.stride_sn];
                    v = dequant1(nib(word, slot), zero_of<FMT>(qz, gn, p.zero_offset), s);
                }
                bv[i] = v;
            }
            __syncthreads();   // previous iteration's MFMA reads are done
            *reinterpret_cast<e8_t*>(&As[a_row][a_k]) =
                e8_t{av[0], av[1], av[2], av[3], av[4], av[5], av[6], av[7]};
            *reinterpret_cast<e8_t*>(&Bs[b_col][b_k]) =
                e8_t{bv[0], bv[1], bv[2], bv[3], bv[4], bv[5], bv[6], bv[7]};
            __syncthreads();

            // ---- 2 x 2 MFMA 16x16x32 per wave (wave tile 32 x 32)
            const int fr = lane & 15, fk = (lane >> 4) * 8;
            e8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const e8_t*>(&As[wm * 32 + i * 16 + fr][fk]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const e8_t*>(&Bs[wn * 32 + j * 16 + fr][fk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
        }

        // ---- store: lane holds D[4*(lane/16) + r][lane%16]
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
                    const int col = n0 + wn * 32 + j * 16 + (lane & 15);
                    if (row < p.m && col < p.n)
                        pc[(int64_t)row * p.stride_cm + (int64_t)col * p.stride_cn] = (E)acc[i][j][r];
                }
    }
}

}  // namespace w4a16
