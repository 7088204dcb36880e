// Prepared (kernel-native) weight layout and the kernels that read it.
//
// A GPTQ, GPTQ_SYM or AWQ checkpoint (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:15-32,
// awq_gemm_int4_typed.rs:10-31; ferrum's loader ships qweight, scales and qzeros as stored,
// w4a16_gptq_gemm_typed.rs:11-13, :55-60) is rewritten once into one format for all three:
//
//   the matrix is cut into strips of 16 columns; strip s (columns 16 s .. 16 s + 15) is one
//   contiguous run of prep_strip_bytes(K, G) bytes:
//     [table: per block, R = max(1, 128 / G) rows of 16 entries of 32 bits; padded to 256
//      bytes][K/128 blocks of 1 KiB]
//   row r of block kb's table holds group (128 kb / G) + r (G <= 128: the groups of the
//   block's rows in order; G a multiple of 128: the block's one group, repeated for every
//   block in it). Entry c holds that group's fp16 scale for column 16 s + c in its low 16
//   bits and the column's full zero point in its high 16 bits: the GPTQ nibble +
//   zero_offset, 8 for GPTQ_SYM, the AWQ nibble; W16 = RNE_f16((q - z) * s) as in the
//   checkpoint formats (w4a16_gptq_gemm_typed.rs:246-260, awq_gemm_int4_typed.rs:213-228).
//   block kb holds rows 128 kb .. 128 kb + 127 of the strip as 64 lanes x 16 bytes: lane l
//   covers column 16 s + l % 16 and rows 128 kb + 32 (l / 16) + [0, 32), as four 32-bit
//   words of 8 consecutive rows each (word w: rows + 8 w .. + 8 w + 7). Row i of a word sits
//   in nibble slot (i >> 1) | ((i & 1) << 2) (the AWQ slot order), so that
//     (w & 0x000F000F) | 0x64006400        = (1024 + q0, 1024 + q1)
//     (w & 0x00F000F0) | 0x64006400        = (1024 + 16 q2, 1024 + 16 q3)
//     ((w >> 8) & 0x000F000F) | 0x64006400 = (1024 + q4, 1024 + q5)
//     ((w >> 8) & 0x00F000F0) | 0x64006400 = (1024 + 16 q6, 1024 + 16 q7)
//   pair up with the activations (x0, x1) .. (x6, x7) as they lie in memory.
//
// So a workgroup that owns a strip reads one contiguous run of HBM (no 128-byte row segments
// at a stride of N/2 bytes, no separate scale and zero streams; the group table, read first,
// shares DRAM pages with the first blocks), and one workgroup covers the whole K range of its
// 16 columns: the GEMV needs no split-K hand-off at all.
#include "device_common.h"
#include "launch.h"
#include "lds_dma.h"

namespace w4a16 {

// ------------------------------------------------------------------ one-time repack

// Grid (ceil(N / 256), K / 128): a workgroup writes block kb of 16 consecutive strips, thread
// t word t of each (lane t / 4, word t % 4), so its stores are 16 contiguous KiB and it reads
// whole 128-byte lines of the checkpoint (AWQ: 128 rows x 32 words; GPTQ: 16 packed rows x
// 256 columns). With one workgroup per strip the 16 strips sharing a line ran on different
// XCDs and each fetched it: the AWQ repack read 8.7x its input from HBM.
template <int FMT>
__global__ void __launch_bounds__(256)
prep_weights_kernel(const uint32_t* __restrict__ qw, uint32_t* __restrict__ out, int K, int N,
                    uint32_t strip_words, uint32_t table_words) {
    const int kb = blockIdx.y, t = threadIdx.x;
    const int l = t >> 2, w = t & 3;
    const int k0 = 128 * kb + 32 * (l >> 4) + 8 * w;
    for (int si = 0; si < 16; ++si) {
        const int s = 16 * blockIdx.x + si;
        if (16 * s >= N) break;
        const int n = 16 * s + (l & 15);
        uint32_t r = 0;
        if constexpr (FMT == FMT_AWQ) {
            const int NW = N >> 3, sl = awq_slot(n);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t v = qw[(size_t)(k0 + i) * NW + (n >> 3)];
                r |= ((v >> (4 * sl)) & 0xFu) << (4 * prep_slot(i));
            }
        } else {
            const uint32_t v = qw[(size_t)(k0 >> 3) * N + n];
#pragma unroll
            for (int i = 0; i < 8; ++i) r |= ((v >> (4 * i)) & 0xFu) << (4 * prep_slot(i));
        }
        out[(size_t)s * strip_words + table_words + (size_t)kb * 256 + t] = r;
    }
}

// One thread per table entry (block, row, column) of every strip; the same threads also
// clear the table's padding (so the buffer's bytes are a function of the checkpoint alone).
template <int FMT>
__global__ void __launch_bounds__(256)
prep_meta_kernel(const half_t* __restrict__ scales, const uint32_t* __restrict__ qz,
                 uint32_t* __restrict__ out, int K, int N, int G, int zero_offset,
                 uint32_t strip_words) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int R = prep_table_rows(G);
    const uint32_t used = (uint32_t)(K / 128) * (uint32_t)R * 16u, tw = prep_table_words(K, G);
    const uint32_t pad = tw - used;
    if (i < (int64_t)(N / 16) * pad) {
        const int64_t s = i / pad;
        out[s * strip_words + used + (i - s * pad)] = 0u;
    }
    if (i >= (int64_t)(N / 16) * used) return;
    const int s = (int)(i / used), e = (int)(i - (int64_t)s * used);
    const int kb = e / (16 * R), r = (e / 16) % R, n = 16 * s + (e & 15);
    const int g = kb * 128 / G + r;
    uint32_t word = 0;
    if constexpr (FMT != FMT_GPTQ_SYM) word = qz[(size_t)g * (N >> 3) + (n >> 3)];
    const uint32_t z = (uint32_t)zero_of<FMT>(word, n, zero_offset);
    const uint32_t sc = __builtin_bit_cast(uint16_t, scales[(size_t)g * N + n]);
    out[(size_t)s * strip_words + e] = sc | (z << 16);
}

hipError_t launch_prepare_layout(int fmt, const uint32_t* qweight, const half_t* scales,
                                 const uint32_t* qzeros, void* out, int K, int N, int G,
                                 int zero_offset, hipStream_t st) {
    (void)hipGetLastError();
    const uint32_t sw = (uint32_t)(prep_strip_bytes(K, G) / 4), tw = prep_table_words(K, G);
    uint32_t* ow = static_cast<uint32_t*>(out);
    const dim3 gw((N + 255) / 256, K / 128);
    const int64_t metas = (int64_t)(N / 16) * tw;   // entries and padding
    const dim3 gm((unsigned)((metas + 255) / 256));
    if (fmt == FMT_AWQ) {
        hipLaunchKernelGGL(prep_weights_kernel<FMT_AWQ>, gw, dim3(256), 0, st, qweight, ow, K, N, sw, tw);
        hipLaunchKernelGGL(prep_meta_kernel<FMT_AWQ>, gm, dim3(256), 0, st, scales, qzeros, ow, K, N, G, zero_offset, sw);
    } else if (fmt == FMT_GPTQ) {
        hipLaunchKernelGGL(prep_weights_kernel<FMT_GPTQ>, gw, dim3(256), 0, st, qweight, ow, K, N, sw, tw);
        hipLaunchKernelGGL(prep_meta_kernel<FMT_GPTQ>, gm, dim3(256), 0, st, scales, qzeros, ow, K, N, G, zero_offset, sw);
    } else {
        hipLaunchKernelGGL(prep_weights_kernel<FMT_GPTQ_SYM>, gw, dim3(256), 0, st, qweight, ow, K, N, sw, tw);
        hipLaunchKernelGGL(prep_meta_kernel<FMT_GPTQ_SYM>, gm, dim3(256), 0, st, scales, qzeros, ow, K, N, G, zero_offset, sw);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ dequant of prepared weights

// W16 = RNE_f16((q - z) * s) for every weight, to [K, N] or (transposed) [N, K]. Grid
// (N / 16, K / 128), one thread per prepared word (8 weights of one column).
__global__ void __launch_bounds__(256)
prep_dequant_kernel(const unsigned char* __restrict__ prep, half_t* __restrict__ out, int K,
                    int N, int G, uint32_t strip_bytes, int transposed) {
    const int s = blockIdx.x, kb = blockIdx.y, t = threadIdx.x;
    const int l = t >> 2, w = t & 3;
    const int n = 16 * s + (l & 15);
    const int k0 = 128 * kb + 32 * (l >> 4) + 8 * w;
    const uint32_t* strip = reinterpret_cast<const uint32_t*>(prep + (size_t)s * strip_bytes);
    const uint32_t word = strip[prep_table_words(K, G) + kb * 256 + t];
    const int R = prep_table_rows(G);
    const uint32_t e = strip[(kb * R + (G < 128 ? (k0 % 128) / G : 0)) * 16 + (l & 15)];
    const half_t sc = __builtin_bit_cast(half_t, (uint16_t)e);
    const int z = (int)(e >> 16);
    half8_t v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = dequant1(nib(word, prep_slot(i)), z, sc);
    if (transposed) {
        *reinterpret_cast<half8_t*>(out + (size_t)n * K + k0) = v;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[(size_t)(k0 + i) * N + n] = v[i];
    }
}

hipError_t launch_prep_dequant(const void* prep, half_t* out, int K, int N, int G, int transposed,
                               hipStream_t st) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(prep_dequant_kernel, dim3(N / 16, K / 128), dim3(256), 0, st,
                       static_cast<const unsigned char*>(prep), out, K, N, G,
                       (uint32_t)prep_strip_bytes(K, G), transposed);
    return hipGetLastError();
}

// ------------------------------------------------------------------ M = 1 GEMV

// One workgroup per strip, W waves over its K / 128 blocks: wave w takes blocks w BPW + j,
// j = 0 .. BPW - 1, so that a wave's activations, table entries and weights are each one
// contiguous range. Order of a lane's loads: the activations of its wave's blocks, their
// table entries, then the blocks (non-temporal). Loads complete in issue order, so x and the
// table have landed while the weights are still arriving, and each block is consumed as it
// lands. Every load is issued unconditionally: offsets past the end of their buffer resource
// read zero without touching memory, and a block past the end of the strip (weights, x and
// scale all zero) adds exactly zero, so no wave branches on its block count.
//
// Each wave stages what its own blocks need in a private LDS region (no wave waits for
// another before its block loop; the workgroup meets once, to add its waves' sums). The
// activations are stored as 80-byte rows of 32 rows of x: a block's four rows are 80 bytes
// apart and fall in disjoint banks.
constexpr int PREP_SEG_BYTES = 80;

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// v summed over the 4 lanes of its quad (DPP quad permutations)
__device__ __forceinline__ float quad_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    return v;
}

// v summed over the 16 lanes of its row (DPP row rotations, then quad permutations)
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
    return quad_sum(v);
}

// Matrix-core kernel (G % 128 == 0, so a block lies in one group). A prepared word is
// exactly a B operand of v_mfma_f32_16x16x32_f16 after one shift and four v_and_or_b32:
// lane l supplies column l % 16 and rows 8 (l / 16) + e, e = 0..7, of the MFMA's 32-row
// step; step st of block kb takes word st of every lane, i.e. rows 128 kb + 32 h + 8 st + e
// (h = l / 16), and the A operand of lane l is x at the same rows. The B values are
// 1024 + c_e q_e with c_e = 1, 1, 16, 16, 1, 1, 16, 16 (the exponent trick without the
// shifts the odd pairs would need), so A carries x'_e = x_e / c_e (a power-of-two scaling,
// exact in fp16 down to the subnormal range), and
//   D = sum_k x'_k (1024 + c_k q_k) = 1024 S' + sum_k x_k q_k,
//   S' = sum_k x'_k, S = sum_k x_k over the block,
// so y += s (D - 1024 S' - z S) = s sum_k x_k (q_k - z). Every row of A is the same x', so
// every row of D holds the result and each lane keeps the sum of its column. VALU per 8
// weights: one shift and four v_and_or_b32.
// LDS per wave: BPW x 4 rows of x'; BPW float pairs (1024 S', S); BPW x 16 table entries.
template <int BPW>
constexpr size_t prep_mfma_wave_lds() { return (size_t)BPW * (4 * PREP_SEG_BYTES + 8 + 16 * 4); }

template <int BPW>
__global__ void __launch_bounds__(1024)
gemv_prep_mfma_kernel(PrepParams p) {
    // 16-byte chunks of x per lane (16 per block) and (block, column) table entries per
    // lane (16 per block); with BPW = 2 only lanes 0..31 load them
    constexpr int XC = BPW >= 4 ? BPW / 4 : 1;
    constexpr int EC = BPW >= 4 ? BPW / 4 : 1;
    static_assert(BPW == 2 || BPW % 4 == 0, "blocks per wave");
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int W = blockDim.x >> 6;
    const int s = blockIdx.x;
    const int blocks = p.K >> 7;
    const unsigned char* strip = p.prep + (size_t)s * p.strip_bytes;
    const uint32_t tbytes = prep_table_words(p.K, p.G) * 4u;
    unsigned char* xs = lds + (size_t)wave * prep_mfma_wave_lds<BPW>();        // BPW x 4 rows
    float2* bsum = reinterpret_cast<float2*>(xs + BPW * 4 * PREP_SEG_BYTES);   // BPW
    uint32_t* tab = reinterpret_cast<uint32_t*>(bsum + BPW);                    // BPW x 16
    float* red = reinterpret_cast<float*>(lds + (size_t)W * prep_mfma_wave_lds<BPW>());

    // ---- loads: the x of the wave's blocks, their table entries, then the blocks
    const bufrsrc_t xr = make_rsrc(p.x, (uint32_t)p.K * 2u);
    const bufrsrc_t tr = make_rsrc(strip, tbytes);
    const bufrsrc_t wr = make_rsrc(strip + tbytes, (uint32_t)p.K * 8u);
    u32x4 xv[XC], wv[BPW];
    uint32_t ev[EC];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = lane + 64 * i, kb = wave * BPW + (c >> 4);   // chunk c: block c / 16 of the wave
        const uint32_t off = kb < blocks && c < 16 * BPW ? (uint32_t)(kb * 128 + (c & 15) * 8) * 2u
                                                         : (uint32_t)p.K * 2u;
        xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }
    {   // the wave's BPW x 16 entries are contiguous: EC consecutive ones per lane, one load
        // (streaming: with the default policy the same entries cost 0.3 us more per call)
        const uint32_t off = EC * lane < 16 * BPW ? (uint32_t)(wave * BPW * 16 + EC * lane) * 4u : tbytes;
        if constexpr (EC == 1) {
            ev[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(tr, off, 0, 2);
        } else if constexpr (EC == 2) {
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(tr, off, 0, 2));
            ev[0] = v.x; ev[1] = v.y;
        } else {
            const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(tr, off, 0, 2));
            ev[0] = v.x; ev[1] = v.y; ev[2] = v.z; ev[3] = v.w;
        }
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const uint32_t off = (uint32_t)(wave * BPW + j) * 1024u + (uint32_t)lane * 16u;
        wv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2));
    }

    // ---- stage x' (odd pairs / 16), the per-block sums and the table entries
    const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
    const half2_t s16 = {(half_t)(1.0f / 16.0f), (half_t)(1.0f / 16.0f)};
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = lane + 64 * i;              // block c / 16, row c / 4 of the region
        const u32x4 v = xv[i];
        const half2_t a0 = as_h2(v.x), a2 = as_h2(v.z);
        const half2_t a1 = as_h2(v.y) * s16, a3 = as_h2(v.w) * s16;
        const float sp = row16_sum(dot2(a0, one2, dot2(a1, one2, dot2(a2, one2, dot2(a3, one2, 0.f)))));
        const float sx = row16_sum(dot2(a0, one2, dot2(as_h2(v.y), one2, dot2(a2, one2, dot2(as_h2(v.w), one2, 0.f)))));
        if (c < 16 * BPW) {
            unsigned char* row = xs + (size_t)(c >> 2) * PREP_SEG_BYTES;
            *reinterpret_cast<u32x4*>(row + (c & 3) * 16) = u32x4{as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)};
            if ((c & 15) == 0) bsum[c >> 4] = make_float2(1024.0f * sp, sx);
        }
    }
#pragma unroll
    for (int i = 0; i < EC; ++i)
        if (EC * lane + i < 16 * BPW) tab[EC * lane + i] = ev[i];
    // the region is this wave's alone: its LDS writes are ordered before its reads below

    // ---- blocks: four MFMAs each
    const int col = lane & 15, h = lane >> 4;
    float y = 0.f;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const unsigned char* row = xs + (size_t)(j * 4 + h) * PREP_SEG_BYTES;
        const float2 bx = bsum[j];
        const uint32_t e = tab[j * 16 + col];
        float4_t d = {0.f, 0.f, 0.f, 0.f};
        const uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const half8_t a = *reinterpret_cast<const half8_t*>(row + 16 * st);
            const uint32_t q = wd[st], q8 = q >> 8;
            const u32x4 bw = {as_u32(nib_pair(q)), as_u32(nib_pair16(q)), as_u32(nib_pair(q8)),
                              as_u32(nib_pair16(q8))};
            d = mfma16x16x32(a, __builtin_bit_cast(half8_t, bw), d);
        }
        const float sc = (float)__builtin_bit_cast(half_t, (uint16_t)e), z = (float)(e >> 16);
        y = __builtin_fmaf(sc, d[0] - __builtin_fmaf(z, bx.y, bx.x), y);
    }

    // ---- reduce over the waves (every lane of a column holds the same sum)
    if (lane < 16) red[wave * 16 + lane] = y;
    __syncthreads();
    if (t < 16) {
        float acc = 0.f;
        for (int w = 0; w < W; ++w) acc += red[w * 16 + t];
        p.out[(size_t)s * 16 + t] = (half_t)acc;
    }
}

// VALU kernel for group sizes 32 and 64 (a block then spans groups; a lane's 32 rows still
// lie in one). Per lane and block:
//   A = sum_i x_i (1024 + c_i q_i), c_i = 1 or 16 by pair (the exponent trick above),
//   y += s * (A_1 + A_16 / 16 - (1024 X_1 + 64 X_16) - z (X_1 + X_16))
// where X_1, X_16 are the sums of x over the rows of each kind, computed per 32-row segment
// while x is staged and kept in the 16 bytes that pad the segment's row. Each lane loads the
// table entry of its own (segment, column) for every block. The four lanes of a column
// (l, l+16, l+32, l+48) and the waves are then reduced.
template <int BPW>
constexpr size_t prep_valu_wave_lds() { return (size_t)BPW * 4 * PREP_SEG_BYTES; }

template <int BPW>
__global__ void __launch_bounds__(1024)
gemv_prep_valu_kernel(PrepParams p) {
    constexpr int XC = BPW / 4;
    static_assert(BPW % 4 == 0, "blocks per wave");
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int W = blockDim.x >> 6;
    const int s = blockIdx.x;
    const int blocks = p.K >> 7;
    const int col = lane & 15, h = lane >> 4;
    const unsigned char* strip = p.prep + (size_t)s * p.strip_bytes;
    const uint32_t tbytes = prep_table_words(p.K, p.G) * 4u;
    unsigned char* xs = lds + (size_t)wave * prep_valu_wave_lds<BPW>();
    float* red = reinterpret_cast<float*>(lds + (size_t)W * prep_valu_wave_lds<BPW>());

    const bufrsrc_t xr = make_rsrc(p.x, (uint32_t)p.K * 2u);
    const bufrsrc_t tr = make_rsrc(strip, tbytes);
    const bufrsrc_t wr = make_rsrc(strip + tbytes, (uint32_t)p.K * 8u);
    u32x4 xv[XC], wv[BPW];
    uint32_t ev[BPW];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = lane + 64 * i, kb = wave * BPW + (c >> 4);
        const uint32_t off = kb < blocks ? (uint32_t)(kb * 128 + (c & 15) * 8) * 2u : (uint32_t)p.K * 2u;
        xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const int kb = wave * BPW + j;
        // table row of this lane's 32 rows: (32 h) / G of the block's R = 128 / G rows
        const uint32_t off = kb < blocks ? ((uint32_t)(kb * (128 / p.G) + 32 * h / p.G) * 16u + (uint32_t)col) * 4u : tbytes;
        ev[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(tr, off, 0, 2);
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const uint32_t off = (uint32_t)(wave * BPW + j) * 1024u + (uint32_t)lane * 16u;
        wv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2));
    }

    // ---- stage x with the per-segment sums
    const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = lane + 64 * i;              // segment c / 4 of the region, quarter c % 4
        const u32x4 v = xv[i];
        const float x1 = quad_sum(dot2(as_h2(v.x), one2, dot2(as_h2(v.z), one2, 0.f)));    // rows 0,1,4,5
        const float x16 = quad_sum(dot2(as_h2(v.y), one2, dot2(as_h2(v.w), one2, 0.f)));   // rows 2,3,6,7
        unsigned char* row = xs + (size_t)(c >> 2) * PREP_SEG_BYTES;
        *reinterpret_cast<u32x4*>(row + (c & 3) * 16) = v;
        if ((c & 3) == 0)
            *reinterpret_cast<float2*>(row + 64) = make_float2(1024.0f * x1 + 64.0f * x16, x1 + x16);
    }

    float y = 0.f;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const unsigned char* row = xs + (size_t)(j * 4 + h) * PREP_SEG_BYTES;
        const float2 bx = *reinterpret_cast<const float2*>(row + 64);
        float a1 = 0.f, a16 = 0.f;
        const uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x4 xq = *reinterpret_cast<const u32x4*>(row + 16 * w);
            const uint32_t d = wd[w], d8 = d >> 8;
            a1 = dot2(nib_pair(d), as_h2(xq.x), a1);
            a16 = dot2(nib_pair16(d), as_h2(xq.y), a16);
            a1 = dot2(nib_pair(d8), as_h2(xq.z), a1);
            a16 = dot2(nib_pair16(d8), as_h2(xq.w), a16);
        }
        const float sc = (float)__builtin_bit_cast(half_t, (uint16_t)ev[j]), z = (float)(ev[j] >> 16);
        const float u = __builtin_fmaf(a16, 1.0f / 16.0f, a1) - __builtin_fmaf(z, bx.y, bx.x);
        y = __builtin_fmaf(sc, u, y);
    }

    y += shfl_xor_f(y, 16);
    y += shfl_xor_f(y, 32);
    if (lane < 16) red[wave * 16 + lane] = y;
    __syncthreads();
    if (t < 16) {
        float acc = 0.f;
        for (int w = 0; w < W; ++w) acc += red[w * 16 + t];
        p.out[(size_t)s * 16 + t] = (half_t)acc;
    }
}

// M = 2..4: SPW strips per workgroup over all of K, wave w taking blocks w BPW .. w BPW + BPW
// - 1 of each, with the activations as MFMA A operands read straight from global memory (x is
// a few hundred KiB at most and stays in the caches; SPW strips share each A load). An A
// operand has 16 rows and M <= MP rows are needed, so one A register set carries P = 16 / MP
// blocks: rows [b MP, b MP + MP) hold block b's activations (rows past M repeat row M - 1),
// and the MFMA of block b leaves its result in those rows of D. The zero point is taken out
// of the B operand exactly, (1024 + c q) - (1024 + c z) = c (q - z), c = 1 or 16 as in the
// M = 1 kernel (A carries x / c), so D = sum_k x_k (q_k - z) per block, and y += s D per
// block, strip and row slot; the (wave, slot) sums meet in LDS. VALU per 8 weights: one
// shift, four v_and_or_b32, four v_pk_add_f16. Requires G % 128 == 0 (a block in one group).
template <int MP, int BPW, int SPW>
__global__ void __launch_bounds__(1024)
gemv_prep_rows_kernel(PrepParams p) {
    constexpr int P = 16 / MP, S = BPW / P;
    static_assert(BPW % P == 0 && (BPW == 4 || BPW == 8), "blocks per wave");
    constexpr int EC = BPW / 4;   // table entries per lane per strip (one 32- or 64-bit load)
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int W = blockDim.x >> 6;
    const int s0 = blockIdx.x * SPW;
    const int M = p.M, blocks = p.K >> 7, NS = p.N >> 4;
    const int col = lane & 15, h = lane >> 4;
    const uint32_t tbytes = prep_table_words(p.K, p.G) * 4u;
    const uint32_t pbytes = (uint32_t)NS * p.strip_bytes;
    uint32_t* tab = reinterpret_cast<uint32_t*>(lds) + (size_t)wave * SPW * BPW * 16;
    float* red = reinterpret_cast<float*>(lds + (size_t)W * SPW * BPW * 16 * 4);   // W x P x SPW x M x 16
    const bufrsrc_t xr = make_rsrc(p.x, (uint32_t)M * (uint32_t)p.K * 2u);
    const bufrsrc_t pr = make_rsrc(p.prep, pbytes);
    uint32_t ev[SPW][EC];
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp) {
        // entries of blocks past K read zero (scale 0, zero point 0): their A and B operands
        // are zero too, and 0 x scale must not meet weight bytes read as a scale
        const int s = s0 + sp, e0 = wave * BPW * 16 + EC * lane;
        const uint32_t off = s < NS && e0 / 16 < blocks ? (uint32_t)s * p.strip_bytes + (uint32_t)e0 * 4u : pbytes;
        if constexpr (EC == 1) {
            ev[sp][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, 2);
        } else {
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(pr, off, 0, 2));
            ev[sp][0] = v.x; ev[sp][1] = v.y;
        }
    }
    u32x4 av[S][4], wv[SPW][BPW];
    {
        const int slot = col / MP, r = min(col % MP, M - 1);
#pragma unroll
        for (int a = 0; a < S; ++a) {
            const int kb = wave * BPW + a * P + slot;
            const uint32_t base = kb < blocks ? ((uint32_t)r * (uint32_t)p.K + (uint32_t)(kb * 128 + 32 * h)) * 2u
                                              : (uint32_t)M * (uint32_t)p.K * 2u;
#pragma unroll
            for (int st = 0; st < 4; ++st)
                av[a][st] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, base + 16u * st, 0, 0));
        }
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
            const int s = s0 + sp, kb = wave * BPW + j;
            const uint32_t off = s < NS && kb < blocks
                                     ? (uint32_t)s * p.strip_bytes + tbytes + (uint32_t)kb * 1024u + (uint32_t)lane * 16u
                                     : pbytes;
            wv[sp][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, 2));
        }
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int i = 0; i < EC; ++i) tab[sp * BPW * 16 + EC * lane + i] = ev[sp][i];

    float y[SPW][P][4];
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int b = 0; b < P; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[sp][b][i] = 0.f;
#pragma unroll
    for (int a = 0; a < S; ++a) {
        half8_t A[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const u32x4 v = av[a][st];
            const half2_t h1 = as_h2(v.y) * (half2_t){(half_t)(1.0f / 16.0f), (half_t)(1.0f / 16.0f)};
            const half2_t h3 = as_h2(v.w) * (half2_t){(half_t)(1.0f / 16.0f), (half_t)(1.0f / 16.0f)};
            A[st] = __builtin_bit_cast(half8_t, u32x4{v.x, as_u32(h1), v.z, as_u32(h3)});
        }
#pragma unroll
        for (int b = 0; b < P; ++b) {
            const int j = a * P + b;
#pragma unroll
            for (int sp = 0; sp < SPW; ++sp) {
                const uint32_t e = tab[sp * BPW * 16 + j * 16 + col];
                const uint32_t z = e >> 16;
                const uint32_t ze = ((0x6400u + z) * 0x10001u) | 0x80008000u;
                const uint32_t zo = ((0x6400u + 16u * z) * 0x10001u) | 0x80008000u;
                float4_t d = {0.f, 0.f, 0.f, 0.f};
                const uint32_t wd[4] = {wv[sp][j].x, wv[sp][j].y, wv[sp][j].z, wv[sp][j].w};
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const uint32_t q = wd[st], q8 = q >> 8;
                    const u32x4 bw = {as_u32(nib_pair(q) + as_h2(ze)), as_u32(nib_pair16(q) + as_h2(zo)),
                                      as_u32(nib_pair(q8) + as_h2(ze)), as_u32(nib_pair16(q8) + as_h2(zo))};
                    d = mfma16x16x32(A[st], __builtin_bit_cast(half8_t, bw), d);
                }
                const float sc = (float)__builtin_bit_cast(half_t, (uint16_t)e);
#pragma unroll
                for (int i = 0; i < 4; ++i) y[sp][b][i] = __builtin_fmaf(sc, d[i], y[sp][b][i]);
            }
        }
    }
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int b = 0; b < P; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * h + i - b * MP;
                if (m >= 0 && m < MP && m < M) red[(((wave * P + b) * SPW + sp) * M + m) * 16 + col] = y[sp][b][i];
            }
    __syncthreads();
    for (int o = t; o < SPW * M * 16; o += blockDim.x) {
        const int sp = o / (M * 16), rem = o - sp * M * 16;
        if (s0 + sp >= NS) continue;
        float acc = 0.f;
        for (int wb = 0; wb < W * P; ++wb) acc += red[(wb * SPW + sp) * M * 16 + rem];
        p.out[(size_t)(rem >> 4) * p.N + (size_t)(s0 + sp) * 16 + (rem & 15)] = (half_t)acc;
    }
}

// M <= 64 (small batches): A operand st of 16-row tile tt of block kb holds, in lane l, x at
// row 16 tt + l % 16 and rows 128 kb + 32 (l / 16) + 8 st + [0, 8), the rows the prepared
// word st of lane l covers on the B side. Rows of a tile past M are zero.
//
// One workgroup owns S strips over the whole K range: wave w takes blocks w BPW .. w BPW +
// BPW - 1 (so no split-K hand-off and no partial sums leave the CU); its table entries and
// weights run PD blocks ahead of its MFMAs. Per block and strip, B = word st of the lane's
// 16 bytes as eight fp16 q - z: ((w >> 4 i) & 0x000F000F | 0x64006400) - (1024 + z) is exact;
// one chain of four MFMAs per 16-row tile gives D = sum_k x_k (q_k - z) over the block, and
// y += s D. The waves' sums meet in LDS and are added in wave order.
// Requires G % 128 == 0 and fewer than 2^31 bytes of prepared weights.
//
// x is read as stored ([M, K], row-major) and put in that order on the way into LDS, so no
// pass over x runs before the kernel. Per block and 16-row tile a wave issues four
// LDS-DMA loads of 1 KiB (buffer_load_dwordx4 ... lds: lane i's 16 bytes land at the wave's
// base + 16 i), load q covering rows 4 q .. 4 q + 3 of the tile: lane i reads row
// r = 4 q + i / 16, chunk c = (i % 16) ^ r of the block's 256 bytes (chunk c: the row's x at
// 8 c .. 8 c + 7), so each load is four whole 256-byte row segments and chunk c of row r sits
// at r * 256 + (c ^ r) * 16 of the tile's 4 KiB. The A operand of step st is chunk
// 4 (l / 16) + st of row l % 16: one ds_read_b128 per lane, the 16 lanes of a row group at 16
// distinct positions (no bank conflicts).
// The x loads go through the compiler's buffer-load-to-LDS builtin, so its own waits for the
// table and weight loads count them; it does not order LDS reads after them, so the kernel
// waits for them itself (vmcnt: the loads issued after a block's x loads may still be in
// flight) before reading a block's x.
//   XD = 1 (one 16-row tile, every block of the wave loaded up front, PD = BPW): all the x
//   loads go first, then the table and weight loads; one wait (vmcnt 2 S BPW) precedes the
//   first LDS read.
//   XD = 2 (any tile count): R = xd_slots(MT) slots of MT x 4 KiB per wave, x running R
//   blocks ahead: block j + R's x is loaded into block j's slot as soon as block j's A
//   operands are in registers (lgkmcnt(0) first), and block j's wait counts the loads issued
//   after its x loads (xd_after).
// Slots of x per wave in the streamed XD mode: 4 KiB per tile and slot, 8 waves at most
constexpr int xd_slots(int MT) { return MT == 1 ? 4 : MT == 2 ? 2 : 1; }

// Streamed XD mode: VMEM loads issued after block j's x loads by the time block j is read.
// Issue order: the x of blocks 0 .. R - 1, then the table and weight loads (lops each) of
// blocks 0 .. PD - 1; iteration i then issues the x of block i + R (dops loads) and the
// table and weights of block i + PD, each while that block exists.
constexpr int xd_after(int j, int R, int PD, int BPW, int dops, int lops) {
    int n = 0, i = 0;
    if (j < R) {
        n = ((R < BPW ? R : BPW) - 1 - j) * dops + PD * lops;
    } else {
        if (j - R + PD < BPW) n = lops;
        i = j - R + 1;
    }
    for (; i < j; ++i) {
        if (i + R < BPW) n += dops;
        if (i + PD < BPW) n += lops;
    }
    return n < 0 ? 0 : n < 63 ? n : 63;
}

// s_waitcnt vmcnt(xd_after(j, ...)) for a j that is a constant once the caller's loop is
// unrolled: the count is the same for every block from R until R + PD blocks before the end,
// so a few branches (folded away per iteration) cover every j. R, PD <= 4.
template <int R, int PD, int BPW, int DOPS, int LOPS>
__device__ __forceinline__ void xd_wait(const int j) {
    static_assert(R <= 4 && PD <= 4, "xd_wait cases");
#define W4A16_XDW(jj) wait_vmcnt<xd_after((jj), R, PD, BPW, DOPS, LOPS)>()
    if (j < R) {
        switch (j) {
            case 0: W4A16_XDW(0); break;
            case 1: W4A16_XDW(1); break;
            case 2: W4A16_XDW(2); break;
            default: W4A16_XDW(3); break;
        }
    } else if (j < BPW - R - PD) {
        W4A16_XDW(R);
    } else {
        switch (BPW - 1 - j) {
            case 0: W4A16_XDW(BPW - 1); break;
            case 1: W4A16_XDW(BPW - 2); break;
            case 2: W4A16_XDW(BPW - 3); break;
            case 3: W4A16_XDW(BPW - 4); break;
            case 4: W4A16_XDW(BPW - 5); break;
            case 5: W4A16_XDW(BPW - 6); break;
            case 6: W4A16_XDW(BPW - 7); break;
            default: W4A16_XDW(BPW - 8); break;
        }
    }
#undef W4A16_XDW
}

// Weight sources of the small-batch kernel: the prepared layout, or a GPTQ checkpoint as stored
// (qweight [K/8, N], scales [K/G, N], qzeros [K/G, N/8]; GPTQ_SYM: zero 8). For the checkpoint
// a workgroup owns 16 S consecutive columns and lane l of sub-block s holds column
// n0 + S (l % 16) + s (the MFMA's column order is free as long as the output follows it):
// a lane loads S consecutive words of each packed row (16 lanes: 64 S contiguous bytes of the
// row), its S scales in one load and its zero word in one. Word st of a lane's block is
// packed row 16 kb + 4 (l / 16) + st, i.e. rows 128 kb + 32 (l / 16) + 8 st + [0, 8), the
// rows the A operand of step st holds; GPTQ packs row 8 r + i in nibble i, so the pair
// (i, i + 1) = ((w >> 4 i) & 0xF, (w >> 4 i + 4) & 0xF) becomes the fp16 pair
// (1024 + q_i, 1024 + q_i+1) with one shift each and two v_and_or_b32. The checkpoint kernel
// then forms each weight as the reference does, W16 = RNE_f16((q - z) s) (v_pk_add_f16 of
// -(1024 + z), exact, then v_pk_mul_f16), and the MFMA chain accumulates x W16 in fp32; the
// prepared kernel scales each block's sum of x (q - z) in fp32 instead.
//
// Act-order (SRC_GPTQ_ACT, SRC_SYM_ACT: g_idx gives each row's group): the workgroup first
// builds an LDS table of (scale | fp16(1024 + z) << 16) for every group and each of its 16 S
// columns, and the rows' table offsets (clamp(g_idx, 0, K/G - 1) * 16 S) for all of K; the
// loads for both are issued ahead of x and the weights, so they land first. A lane's B
// operand of step st then takes, per row pair, its two entries per column: v_perm_b32
// assembles the pairs (1024 + z0, 1024 + z1) and (s0, s1), and W16 = RNE_f16((q - z) s)
// as before (the weights stay bit-exact; any group size).
//
// Prepared act-order (SRC_PREP_ACT): the prepared layout of an act-order checkpoint as stored
// (rows in their own order, g_idx gives each row's group). The strip's inline table holds every
// group's (scale, full zero point) already (table row g (G / 128) for G >= 128, row g for G =
// 32 or 64), so the workgroup's LDS table is filled from it, and the B operand is formed per
// row pair as for the checkpoint (W16 = RNE_f16((q - z) s), accumulated in the MFMA chain)
// from the prepared words (row pair (2 i, 2 i + 1) in nibble slots i and i + 4). The lane's S
// strips sit at table positions S col + s, so its S entries are one read as for the checkpoint.
constexpr int SRC_PREP = 0, SRC_GPTQ = 1, SRC_GPTQ_SYM = 2, SRC_GPTQ_ACT = 3, SRC_SYM_ACT = 4,
              SRC_PREP_ACT = 5;
// act-order: table entries per thread (4 columns of one group per pass, ACT_TI passes) and
// g_idx rows per thread (two 16-byte loads): at most 4096 entries and K <= 4096
constexpr int ACT_TI = 2, ACT_MAX_ENTRIES = 4 * 512 * ACT_TI, ACT_MAX_K = 8 * 512;

__device__ __forceinline__ uint32_t gptq_pair(uint32_t w, int i) {   // i even, constant
    const uint32_t x = w >> (4 * i);
    return (x & 0xFu) | ((x << 12) & 0xF0000u) | 0x64006400u;
}

template <int S> struct ck_words;
template <> struct ck_words<1> { typedef uint32_t type; };
template <> struct ck_words<2> { typedef u32x2 type; };
template <> struct ck_words<4> { typedef u32x4 type; };

// S consecutive 32-bit words at byte offset off; ck_load<0>: one 16-bit value
template <int S>
__device__ __forceinline__ typename ck_words<S ? S : 1>::type ck_load(bufrsrc_t r, uint32_t off) {
    if constexpr (S == 0) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2);
    else if constexpr (S == 1) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 2);
    else if constexpr (S == 2) return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2));
    else return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
template <int S>
__device__ __forceinline__ uint32_t ck_word(const typename ck_words<S>::type& v, int s) {
    if constexpr (S == 1) return v;
    else return v[s];
}

template <int MT, int S, int BPW, int PD, int XD, int SRC = SRC_PREP>
__global__ void __launch_bounds__(512)
gemm_prep_frag_kernel(PrepFragParams p) {
    constexpr bool PA = SRC == SRC_PREP_ACT;   // prepared strips with g_idx
    constexpr bool CK = SRC != SRC_PREP && !PA;   // checkpoint tensors as stored
    constexpr bool ACT = SRC == SRC_GPTQ_ACT || SRC == SRC_SYM_ACT || PA;
    constexpr bool W16 = CK || ACT;   // W16 formed per weight, accumulated in the MFMA chain
    constexpr bool ZQ = SRC == SRC_GPTQ || SRC == SRC_GPTQ_ACT;    // zero points from qzeros
    // loads per block besides x: the table entries and weights of S strips (prepared); four
    // words, the scales and the zero word (checkpoint); four words (act-order); the weights of
    // S strips (prepared act-order)
    constexpr int LOPS = PA ? S : ACT ? 4 : CK ? (SRC == SRC_GPTQ ? 6 : 5) : 2 * S;
    static_assert(PD >= 1 && PD <= BPW, "prefetch depth");
    static_assert(XD == 2 || (XD == 1 && MT == 1 && PD == BPW && LOPS * BPW <= 63),
                  "XD 1: one tile, all blocks up front");
    static_assert(!CK || S == 1 || S == 2 || S == 4, "checkpoint: 1, 2 or 4 columns per lane");
    constexpr int R = XD == 2 ? xd_slots(MT) : 1;   // XD 2: slots of x per wave
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int W = blockDim.x >> 6;
    const int col = lane & 15, h = lane >> 4;
    const int NS = p.N >> 4, KB = p.K >> 7, M = p.M;
    const int s0 = blockIdx.x * S;             // prepared: first strip
    const int n0 = blockIdx.x * 16 * S;        // checkpoint: first column
    const int nc = n0 + S * col;               // checkpoint: the lane's first column
    const uint32_t tbytes = CK ? 0u : prep_table_words(p.K, p.G) * 4u;
    const uint32_t pbytes = CK ? 0u : (uint32_t)NS * p.strip_bytes;
    const bufrsrc_t pr = make_rsrc(CK ? nullptr : p.prep, pbytes);
    const uint32_t qbytes = CK ? (uint32_t)(p.K / 8) * (uint32_t)p.N * 4u : 0u;
    const uint32_t sbytes = CK ? (uint32_t)(p.K / p.G) * (uint32_t)p.N * 2u : 0u;
    const uint32_t zbytes = ZQ ? (uint32_t)(p.K / p.G) * (uint32_t)(p.N / 8) * 4u : 0u;
    const bufrsrc_t qr = make_rsrc(CK ? p.qweight : nullptr, qbytes);
    const bufrsrc_t sr = make_rsrc(CK ? p.scales : nullptr, sbytes);
    const bufrsrc_t zr = make_rsrc(ZQ ? p.qzeros : nullptr, zbytes);
    const int bpg = CK && p.G >= 128 ? p.G / 128 : 1;   // checkpoint: blocks per group (plain order: G % 128 == 0)
    const bufrsrc_t xrs = make_rsrc(p.x, (uint32_t)M * (uint32_t)p.K * 2u);
    // XD 1: the wave's x, block j at 4 KiB j; XD 2: its R slots, block j's tile tt at
    // ((j % R) MT + tt) 4 KiB
    unsigned char* xw = lds + (size_t)wave * (XD == 1 ? BPW * 4096 : R * MT * 4096);
    (void)pr; (void)qr; (void)sr; (void)zr; (void)bpg; (void)nc; (void)s0; (void)n0; (void)tbytes;

    // act-order: the table [K/G][16 S] and the rows' offsets into it [K], after the waves' x
    constexpr int WN = 16 * S;
    const int NG = p.K / p.G;
    uint32_t* tab = reinterpret_cast<uint32_t*>(lds + (size_t)W * (XD == 1 ? BPW * 4096 : R * MT * 4096));
    int* gof = reinterpret_cast<int*>(tab + (ACT ? NG * WN : 0));
    (void)tab; (void)gof;
    u32x2 tsv[ACT ? ACT_TI : 1];
    uint32_t tzv[ACT ? ACT_TI : 1];
    uint32_t pev[PA ? ACT_TI : 1][PA ? 4 : 1];
    u32x4 giv[ACT ? 2 : 1];
    (void)tsv; (void)tzv; (void)pev; (void)giv;
    if constexpr (ACT) {
        // issued first: pass i of thread t covers table positions 4 q .. 4 q + 3 of group g,
        // u = t + 512 i = g (WN / 4) + q (checkpoint: columns n0 + 4 q + c; prepared: position
        // S col + s = strip s0 + s, column col); then g_idx rows 8 t .. 8 t + 7
        const bufrsrc_t gr = make_rsrc(p.g_idx, (uint32_t)p.K * 4u);
        const int trows = p.G >= 128 ? p.G / 128 : 1;   // prepared: table rows per group step
#pragma unroll
        for (int i = 0; i < ACT_TI; ++i) {
            const int u = t + 512 * i, g = u / (WN / 4), q = u - g * (WN / 4);
            const bool in = g < NG;
            if constexpr (PA) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int pos = 4 * q + c, strip = s0 + pos % S, cl = pos / S;
                    pev[i][c] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                        pr, in && strip < NS ? (uint32_t)strip * p.strip_bytes + (uint32_t)(g * trows * 16 + cl) * 4u
                                             : pbytes, 0, 0);
                }
            } else {
                tsv[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                    sr, in ? (uint32_t)(g * p.N + n0 + 4 * q) * 2u : sbytes, 0, 0));
                if constexpr (ZQ)
                    tzv[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                        zr, in ? (uint32_t)(g * (p.N >> 3) + ((n0 + 4 * q) >> 3)) * 4u : zbytes, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            giv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, (uint32_t)(8 * t + 4 * i) * 4u, 0, 0));
    }

    // prepared: ev = table entries, wv = 16-byte lane chunks (one per strip); checkpoint:
    // ev[j][0] = the zero word, cs = the lane's S scales (raw), cw = word st of every column
    uint32_t ev[BPW][S];
    u32x4 wv[CK ? 1 : BPW][S];
    typename ck_words<CK ? S : 1>::type cw[CK ? BPW : 1][4];
    typename ck_words<CK ? (S + 1) / 2 : 1>::type cs[CK ? BPW : 1];   // S = 1: one 16-bit load
    (void)wv; (void)cw; (void)cs;
    auto load = [&](const int j) __attribute__((always_inline)) {
        const int kb = wave * BPW + j;
        const bool kin = kb < KB;
        if constexpr (CK) {
            const int g = kb / bpg;
            const uint32_t so = kin ? (uint32_t)(g * p.N + nc) * 2u : sbytes;
            if constexpr (!ACT) cs[j] = ck_load<S / 2>(sr, so);
            if constexpr (SRC == SRC_GPTQ)
                ev[j][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    zr, kin ? (uint32_t)(g * (p.N >> 3) + (nc >> 3)) * 4u : zbytes, 0, 2);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const uint32_t off = kin ? ((uint32_t)(16 * kb + 4 * h + st) * (uint32_t)p.N + (uint32_t)nc) * 4u
                                         : qbytes;
                cw[j][st] = ck_load<S>(qr, off);
            }
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                if constexpr (PA) break;   // the entries come from the LDS table
                const int strip = s0 + s;
                const uint32_t off = kin && strip < NS ? (uint32_t)strip * p.strip_bytes + (uint32_t)(kb * 16 + col) * 4u
                                                       : pbytes;
                ev[j][s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, 2);
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int strip = s0 + s;
                const uint32_t off = kin && strip < NS
                                         ? (uint32_t)strip * p.strip_bytes + tbytes + (uint32_t)kb * 1024u + (uint32_t)lane * 16u
                                         : pbytes;
                wv[j][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, 2));
            }
        }
    };
    // block j's x: MT tiles of 4 KiB from dst. The loads go through the compiler's
    // buffer-load-to-LDS builtin, so its own waits for the table and weight loads count them;
    // it does not order LDS reads after them (the kernel's waits below do), and the empty asm
    // statements keep the loads in the issue order those waits count.
    auto dma_x = [&](const int j, unsigned char* dst) __attribute__((always_inline)) {
        const int kb = wave * BPW + j;
        asm volatile("" ::: "memory");
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = 4 * q + (lane >> 4), m = 16 * tt + r;
                const int c = (lane & 15) ^ r;
                const uint32_t off = kb < KB && m < M ? (uint32_t)(m * p.K + kb * 128 + 8 * c) * 2u : DMA_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    xrs, (__attribute__((address_space(3))) void*)(dst + tt * 4096 + q * 1024), 16, (int)off, 0, 0, 0);
            }
        asm volatile("" ::: "memory");
    };
    if constexpr (XD == 1) {
#pragma unroll
        for (int j = 0; j < BPW; ++j) dma_x(j, xw + j * 4096);
    }
    if constexpr (XD == 2) {
#pragma unroll
        for (int j = 0; j < (R < BPW ? R : BPW); ++j) dma_x(j, xw + j * MT * 4096);
    }
#pragma unroll
    for (int j = 0; j < PD; ++j) load(j);
    if constexpr (ACT) {
        // the act-order table and offsets into LDS (their loads were issued first), then one
        // barrier; the x and weight loads stay in flight
#pragma unroll
        for (int i = 0; i < ACT_TI; ++i) {
            const int u = t + 512 * i, g = u / (WN / 4), q = u - g * (WN / 4);
            if (g < NG) {
                uint32_t e[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if constexpr (PA) {   // prepared entry: scale | full zero point << 16
                        e[c] = (pev[i][c] & 0xFFFFu) | ((0x6400u + (pev[i][c] >> 16)) << 16);
                        continue;
                    }
                    const uint32_t sb = (c & 1 ? tsv[i][c >> 1] >> 16 : tsv[i][c >> 1]) & 0xFFFFu;
                    const uint32_t z = ZQ ? ((tzv[i] >> (4 * ((n0 + 4 * q + c) & 7))) & 0xFu) + (uint32_t)p.zero_offset
                                          : 8u;
                    e[c] = sb | ((0x6400u + z) << 16);
                }
                *reinterpret_cast<u32x4*>(tab + g * WN + 4 * q) = u32x4{e[0], e[1], e[2], e[3]};
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            u32x4 o;
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] = (uint32_t)(min(max((int)giv[i][c], 0), NG - 1) * WN);
            if (8 * t + 4 * i < p.K) *reinterpret_cast<u32x4*>(gof + 8 * t + 4 * i) = o;
        }
        __syncthreads();
    }
    if constexpr (XD == 1) {
        wait_vmcnt<LOPS * BPW>();           // the x loads, issued before every other load
        asm volatile("" ::: "memory");      // the LDS reads below stay after the wait
    }

    // act-order: the lane's 32 row offsets of block j (rows 128 kb + 32 h + [0, 32))
    u32x4 gq[ACT ? 8 : 1];
    (void)gq;
    auto read_gq = [&](const int j) __attribute__((always_inline)) {
        if constexpr (ACT) {
            const int* go = gof + min(wave * BPW + j, KB - 1) * 128 + 32 * h;   // blocks past K add zero x
#pragma unroll
            for (int i = 0; i < 8; ++i) gq[i] = *reinterpret_cast<const u32x4*>(go + 4 * i);
        }
    };
    read_gq(0);

    float acc[S][MT][4];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[s][tt][i] = 0.f;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        u32x4 A[MT][4];
        const int r = lane & 15;
        if constexpr (XD == 2) {
            // block j's x loads are done once only the loads issued after them remain
            xd_wait<R, PD, BPW, 4 * MT, LOPS>(j);
            asm volatile("" ::: "memory");   // the LDS reads below stay after the wait
            const int slot = j % R;
#pragma unroll
            for (int tt = 0; tt < MT; ++tt)
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    A[tt][st] = *reinterpret_cast<const u32x4*>(xw + (slot * MT + tt) * 4096 + r * 256 +
                                                                (((4 * h + st) ^ r) << 4));
            if (j + R < BPW) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the slot's reads are done
                dma_x(j + R, xw + slot * MT * 4096);
            }
        }
        if (j + PD < BPW) load(j + PD);
        if constexpr (XD == 1) {
#pragma unroll
            for (int st = 0; st < 4; ++st)
                A[0][st] = *reinterpret_cast<const u32x4*>(xw + j * 4096 + r * 256 + (((4 * h + st) ^ r) << 4));
        }
        // act-order: the table entries of the lane's 32 rows, S columns each, through the row
        // offsets read one block ahead (gq), so that no entry read waits on an offset read
        typename ck_words<ACT ? S : 1>::type ent[ACT ? 4 : 1][ACT ? 8 : 1];
        (void)ent;
        if constexpr (ACT) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const uint32_t o[8] = {gq[2 * st].x, gq[2 * st].y, gq[2 * st].z, gq[2 * st].w,
                                       gq[2 * st + 1].x, gq[2 * st + 1].y, gq[2 * st + 1].z, gq[2 * st + 1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    ent[st][e] = *reinterpret_cast<const typename ck_words<S>::type*>(tab + o[e] + S * col);
            }
            if (j + 1 < BPW) read_gq(j + 1);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            // the (scale, zero) of sub-block s and -(1024 + z) as an fp16 pair (exact bits)
            uint32_t zq = 0;
            float sc = 0.f;
            if constexpr (ACT) {
            } else if constexpr (CK) {
                const uint32_t sw = ck_word<(S + 1) / 2>(cs[j], s >> 1);
                sc = (float)__builtin_bit_cast(half_t, (uint16_t)(sw >> (16 * (s & 1))));
                zq = SRC == SRC_GPTQ ? ((ev[j][0] >> (4 * ((nc + s) & 7))) & 0xFu) + (uint32_t)p.zero_offset : 8u;
            } else {
                const uint32_t e = ev[j][s];
                sc = (float)__builtin_bit_cast(half_t, (uint16_t)e);
                zq = e >> 16;
            }
            const half2_t ze = as_h2(((0x6400u + zq) * 0x10001u) | 0x80008000u);
            half8_t B[4];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if constexpr (ACT) {
                    // per row pair: (1024 + z0, 1024 + z1) and (s0, s1) from the two entries
                    uint32_t q;
                    if constexpr (PA) q = wv[j][s][st];
                    else q = ck_word<S>(cw[j][st], s);
                    uint32_t wp[4];
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        const uint32_t e0 = ck_word<S>(ent[st][2 * pp], s), e1 = ck_word<S>(ent[st][2 * pp + 1], s);
                        const half2_t zz = as_h2(perm(e1, e0, 0x07060302u));
                        const half2_t ss = as_h2(perm(e1, e0, 0x05040100u));
                        const half2_t qp = PA ? nib_pair(q >> (4 * pp)) : as_h2(gptq_pair(q, 2 * pp));
                        wp[pp] = as_u32((qp - zz) * ss);
                    }
                    B[st] = __builtin_bit_cast(half8_t, u32x4{wp[0], wp[1], wp[2], wp[3]});
                } else if constexpr (CK) {
                    // W16 = RNE_f16((q - z) s) per weight, as the reference dequantises
                    // (w4a16_gptq_gemm_typed.rs:246-260): q - z exact, one rounded multiply
                    const uint32_t q = ck_word<S>(cw[j][st], s);
                    const half2_t s2 = {(half_t)sc, (half_t)sc};
                    B[st] = __builtin_bit_cast(half8_t, u32x4{as_u32((as_h2(gptq_pair(q, 0)) + ze) * s2),
                                                              as_u32((as_h2(gptq_pair(q, 2)) + ze) * s2),
                                                              as_u32((as_h2(gptq_pair(q, 4)) + ze) * s2),
                                                              as_u32((as_h2(gptq_pair(q, 6)) + ze) * s2)});
                } else {
                    const uint32_t q = wv[j][s][st];
                    B[st] = __builtin_bit_cast(half8_t, u32x4{as_u32(nib_pair(q) + ze), as_u32(nib_pair(q >> 4) + ze),
                                                              as_u32(nib_pair(q >> 8) + ze), as_u32(nib_pair(q >> 12) + ze)});
                }
            }
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                // checkpoint: the dot of x and W16 accumulates in the chain itself; prepared:
                // the block's sum of x (q - z), scaled in fp32
                float4_t d = W16 ? float4_t{acc[s][tt][0], acc[s][tt][1], acc[s][tt][2], acc[s][tt][3]}
                                 : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    d = mfma16x16x32(__builtin_bit_cast(half8_t, A[tt][st]), B[st], d);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[s][tt][i] = W16 ? d[i] : __builtin_fmaf(sc, d[i], acc[s][tt][i]);
            }
        }
    }

    // ---- the waves' sums, added in wave order; lane l of tile tt holds rows 16 tt + 4 (l / 16)
    // + i of column l % 16 of sub-block s
    __syncthreads();   // the sums overwrite other waves' x
    float4_t* red = reinterpret_cast<float4_t*>(lds);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
            red[((wave * S + s) * MT + tt) * 64 + lane] = float4_t{acc[s][tt][0], acc[s][tt][1], acc[s][tt][2], acc[s][tt][3]};
    __syncthreads();
    const float* rf = reinterpret_cast<const float*>(lds);
    for (int o = t; o < S * MT * 256; o += blockDim.x) {
        const int i = o & 3, l = (o >> 2) & 63, rest = o >> 8, tt = rest % MT, s = rest / MT;
        const int m = 16 * tt + 4 * (l >> 4) + i;
        if (m >= M) continue;
        int n;
        if constexpr (CK) {
            n = n0 + S * (l & 15) + s;
        } else {
            if (s0 + s >= NS) continue;
            n = (s0 + s) * 16 + (l & 15);
        }
        float a = 0.f;
        for (int w = 0; w < W; ++w) a += rf[w * S * MT * 256 + o];
        p.out[(size_t)m * p.N + n] = (half_t)a;
    }
}

PrepGemvShape prep_gemv_shape(int M, int N, int K, int G) {
    PrepGemvShape s{};
    if (M < 1 || M > PREP_GEMV_MAX_M || N % 16 || K % 128 || !prep_group_ok(G) || K % G || K > PREP_MAX_K)
        return s;
    const int blocks = K / 128;
    s.mfma = G % 128 == 0;
    if (M > 1) {   // rows kernel: up to 16 waves
        if (!s.mfma || blocks > 8 * 16) return s;
        s.mp = M <= 2 ? 2 : M <= 4 ? 4 : 8;
        // 3..4 rows: 2 strips per workgroup (x read once for both) with 4 blocks per wave where
        // 16 waves cover K: AWQ 4096 -> 14336 M = 3 / 4 8.73 / 9.52 -> 8.48 / 8.92 us; at 2 rows
        // and over longer K it measured no better or slower
        const bool two = s.mp == 4 && blocks <= 4 * 16;
        s.bpw = two ? 4 : 8;
        s.spw = two ? 2 : 1;
        s.waves = (blocks + s.bpw - 1) / s.bpw;
        s.lds = (size_t)s.waves * s.spw * s.bpw * 16 * 4 + (size_t)s.waves * (16 / s.mp) * s.spw * M * 16 * 4;
        s.ok = true;
        return s;
    }
    // blocks per wave: 4 while that fits in 16 waves (more waves, each with a shorter queue of
    // in-order loads: K=4096 -> N=14336 7.11 -> 6.88 us, 4096 -> 4096 3.84 -> 3.69 us against 8
    // blocks per wave), else 8, else 16
    const int bpw = blocks <= 4 * 16 ? 4 : blocks <= 8 * 16 ? 8 : 16;
    const int waves = (blocks + bpw - 1) / bpw;
    s.bpw = bpw;
    s.waves = waves;
    const size_t wave_lds = s.mfma ? (bpw == 16 ? prep_mfma_wave_lds<16>() : bpw == 8 ? prep_mfma_wave_lds<8>()
                                                                                   : prep_mfma_wave_lds<4>())
                                   : (bpw == 16 ? prep_valu_wave_lds<16>() : bpw == 8 ? prep_valu_wave_lds<8>()
                                                                                   : prep_valu_wave_lds<4>());
    s.lds = (size_t)waves * wave_lds + (size_t)waves * 16 * 4;
    s.ok = waves <= 16 && s.lds <= 160 * 1024;
    return s;
}

// Shape of the fragment-order kernel: blocks per wave so that at most 8 waves cover K; S
// strips per workgroup, the most (up to 4; up to 2 from 33 rows or 32 blocks per wave, where
// the registers leave less room) that still gives 192 workgroups (K=4096 -> N=6144: S = 2, 192 workgroups,
// 6.1 us at M = 16 against 7.5 with S = 1; N=14336: S = 4); loads in flight: the whole queue
// at 16 rows when it is 4 blocks, else 2 blocks, then 1 (measured over PD = 1, 2, 4, BPW).
// Blocks per wave, waves, prefetch depth and LDS of the small-batch kernel for s.mt tiles,
// s.s strips (or columns per lane) and K / 128 = KB blocks.
static void frag_common(PrepFragShape& s, int KB) {
    s.bpw = KB <= 32 ? 4 : KB <= 64 ? 8 : KB <= 128 ? 16 : 32;
    s.waves = (KB + s.bpw - 1) / s.bpw;

    s.pd = s.mt == 1 ? (s.bpw == 4 ? 4 : 2) : s.mt == 2 ? 2 : 1;
    // LDS: the waves' x (one 16-row tile and 4 blocks per wave: all of it, 16 KiB per wave;
    // else xd_slots(mt) slots of 4 KiB per tile, at most 128 KiB for 8 waves), later reused
    // for the waves' sums (1 KiB per wave, strip and tile)
    const size_t xl = (size_t)s.waves * (s.mt == 1 && s.bpw == 4 ? 4 : xd_slots(s.mt) * s.mt) * 4096;
    const size_t sums = (size_t)s.waves * s.s * s.mt * 1024;
    s.lds = xl > sums ? xl : sums;
    s.ok = true;
}

PrepFragShape prep_frag_shape(int M, int N, int K, int G, bool act) {
    PrepFragShape s{};
    if (M < 1 || M > PREP_FRAG_MAX_M || N % 16 || K % 128 || K % G || K > PREP_MAX_K)
        return s;
    // plain: G a multiple of 128 (one table entry per block); act-order: any group size of
    // the layout, K within the table's row offsets
    if (act ? (K > ACT_MAX_K || !prep_group_ok(G)) : (G < 128 || G % 128)) return s;
    if (prep_total_bytes(K, N, G) >= ((size_t)1 << 31)) return s;
    const int NS = N / 16, KB = K / 128;
    s.mt = (M + 15) / 16;
    s.s = 1;
    const int bpw = KB <= 32 ? 4 : KB <= 64 ? 8 : KB <= 128 ? 16 : 32;
    for (int c = s.mt <= 2 && bpw <= 16 ? 4 : 2; c > 1; c /= 2)
        if (NS / c >= 192) { s.s = c; break; }
    if (act) {   // as ck_frag_shape: the table of 16 s entries per group
        if (s.mt == 2 && s.s == 4) s.s = 2;
        while (s.s > 1 && (size_t)(K / G) * 16 * s.s > (size_t)ACT_MAX_ENTRIES) s.s /= 2;
        if ((size_t)(K / G) * 16 * s.s > (size_t)ACT_MAX_ENTRIES) return s;
    }
    frag_common(s, KB);
    if (act) {
        s.lds += (size_t)(K / G) * 16 * s.s * 4 + (size_t)K * 4;
        if (s.lds > 160 * 1024) s.ok = false;
    }
    return s;
}

// Checkpoint instances that fit the registers (the others spill: their block loop, with the
// GPTQ unpacking, is not unrolled); fewer columns per lane are tried first
constexpr bool ck_frag_fits(int mt, int s, int bpw) {
    return bpw == 4 || (bpw == 8 && mt * s <= 6) || (bpw == 16 && mt * s <= 2) || (bpw == 32 && mt * s == 1);
}

// The same kernel on a GPTQ / GPTQ_SYM checkpoint as stored: 16 s columns per workgroup, s
// columns per lane (N a multiple of 16 s), G a multiple of 128, fewer than 2^31 bytes per
// tensor.
PrepFragShape ck_frag_shape(int fmt, int M, int N, int K, int G, bool act) {
    PrepFragShape s{};
    if ((fmt != FMT_GPTQ && fmt != FMT_GPTQ_SYM) || M < 1 || M > PREP_FRAG_MAX_M || N % 16 ||
        K % 128 || G < 1 || K % G || K > PREP_MAX_K || (!act && (G < 128 || G % 128)))
        return s;
    if (act && (K > ACT_MAX_K || G % 8)) return s;
    if ((size_t)K / 8 * N * 4 >= ((size_t)1 << 31) || (size_t)K / G * N * 2 >= ((size_t)1 << 31))
        return s;
    const int KB = K / 128;
    s.mt = (M + 15) / 16;
    s.s = 1;
    const int bpw = KB <= 32 ? 4 : KB <= 64 ? 8 : KB <= 128 ? 16 : 32;
    for (int c = s.mt <= 2 && bpw <= 16 ? 4 : 2; c > 1; c /= 2)
        if (N % (16 * c) == 0 && N / (16 * c) >= 192) { s.s = c; break; }
    while (s.s > 1 && !ck_frag_fits(s.mt, s.s, bpw)) s.s /= 2;
    if (!ck_frag_fits(s.mt, s.s, bpw)) return s;
    if (act) {   // the table (4 columns of a group per thread and pass) and the row offsets
        if (s.mt == 2 && s.s == 4) s.s = 2;   // that instance would spill
        while (s.s > 1 && (size_t)(K / G) * 16 * s.s > (size_t)ACT_MAX_ENTRIES) s.s /= 2;
        if ((size_t)(K / G) * 16 * s.s > (size_t)ACT_MAX_ENTRIES || (16 * s.s) % 4) return s;
    }
    frag_common(s, KB);
    if (act) {
        s.lds += (size_t)(K / G) * 16 * s.s * 4 + (size_t)K * 4;
        if (s.lds > 160 * 1024) s.ok = false;
    }
    return s;
}

template <int MT, int S, int BPW, int SRC>
static void launch_frag_inst(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    constexpr int PD1 = MT == 1 ? 2 : MT == 2 ? 2 : 1;   // pd for 8 or more blocks per wave
    const dim3 grid((p.N / 16 + S - 1) / S), block(64 * s.waves);
    // XD 1 with one tile and 4 blocks per wave, else XD 2
    if constexpr (BPW == 4 && MT == 1) hipLaunchKernelGGL((gemm_prep_frag_kernel<1, S, 4, 4, 1, SRC>), grid, block, s.lds, st, p);
    else if constexpr (BPW == 4) hipLaunchKernelGGL((gemm_prep_frag_kernel<MT, S, 4, MT == 2 ? 2 : 1, 2, SRC>), grid, block, s.lds, st, p);
    else hipLaunchKernelGGL((gemm_prep_frag_kernel<MT, S, BPW, PD1, 2, SRC>), grid, block, s.lds, st, p);
}

template <int MT, int S, int SRC>
static hipError_t launch_prep_frag_ms(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    // instances that would not fit the registers: 4 strips over 32 blocks (prepared), and
    // the checkpoint ones ck_frag_fits excludes
    auto fits = [](int bpw) { return SRC == SRC_PREP ? !(S == 4 && bpw == 32) : ck_frag_fits(MT, S, bpw); };
    if (!fits(s.bpw)) return hipErrorInvalidValue;
    if constexpr (SRC == SRC_GPTQ_ACT || SRC == SRC_SYM_ACT || SRC == SRC_PREP_ACT) {   // K <= 4096: 4 blocks per wave
        if (s.bpw != 4) return hipErrorInvalidValue;
        launch_frag_inst<MT, S, 4, SRC>(p, s, st);
        return hipGetLastError();
    } else {
    switch (s.bpw) {
        case 4: launch_frag_inst<MT, S, 4, SRC>(p, s, st); break;
        case 8: if constexpr (SRC == SRC_PREP || ck_frag_fits(MT, S, 8)) { launch_frag_inst<MT, S, 8, SRC>(p, s, st); break; }
                return hipErrorInvalidValue;
        case 16: if constexpr (SRC == SRC_PREP || ck_frag_fits(MT, S, 16)) { launch_frag_inst<MT, S, 16, SRC>(p, s, st); break; }
                 return hipErrorInvalidValue;
        case 32: if constexpr ((SRC == SRC_PREP && S <= 2) || ck_frag_fits(MT, S, 32)) { launch_frag_inst<MT, S, 32, SRC>(p, s, st); break; }
                 return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
    }
}

template <int MT, int SRC>
static hipError_t launch_prep_frag_m(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    switch (s.s) {
        case 1: return launch_prep_frag_ms<MT, 1, SRC>(p, s, st);
        case 2: return launch_prep_frag_ms<MT, 2, SRC>(p, s, st);
        // act-order at 2 row tiles: 2 strips (ck_frag_shape), 4 would spill
        case 4: if constexpr (MT == 1 || (MT == 2 && SRC != SRC_GPTQ_ACT && SRC != SRC_SYM_ACT && SRC != SRC_PREP_ACT))
                    return launch_prep_frag_ms<MT, 4, SRC>(p, s, st);
                [[fallthrough]];
        default: return hipErrorInvalidValue;
    }
}

template <int SRC>
static hipError_t launch_frag_src(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    (void)hipGetLastError();
    if (!s.ok || s.pd != (s.mt == 1 ? (s.bpw == 4 ? 4 : 2) : s.mt == 2 ? 2 : 1)) return hipErrorInvalidValue;
    switch (s.mt) {
        case 1: return launch_prep_frag_m<1, SRC>(p, s, st);
        case 2: return launch_prep_frag_m<2, SRC>(p, s, st);
        case 3: return launch_prep_frag_m<3, SRC>(p, s, st);
        case 4: return launch_prep_frag_m<4, SRC>(p, s, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prep_frag(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    return p.g_idx ? launch_frag_src<SRC_PREP_ACT>(p, s, st) : launch_frag_src<SRC_PREP>(p, s, st);
}

hipError_t launch_ck_frag(int fmt, const PrepFragParams& p, const PrepFragShape& s, hipStream_t st) {
    if (p.g_idx) {
        if (fmt == FMT_GPTQ) return launch_frag_src<SRC_GPTQ_ACT>(p, s, st);
        if (fmt == FMT_GPTQ_SYM) return launch_frag_src<SRC_SYM_ACT>(p, s, st);
        return hipErrorInvalidValue;
    }
    if (fmt == FMT_GPTQ) return launch_frag_src<SRC_GPTQ>(p, s, st);
    if (fmt == FMT_GPTQ_SYM) return launch_frag_src<SRC_GPTQ_SYM>(p, s, st);
    return hipErrorInvalidValue;
}

template <int BPW>
static void launch_prep_m1_b(const PrepParams& p, const PrepGemvShape& s, hipStream_t st) {
    const dim3 grid(p.N / 16), block(64 * s.waves);
    if (s.mfma) hipLaunchKernelGGL((gemv_prep_mfma_kernel<BPW>), grid, block, s.lds, st, p);
    else hipLaunchKernelGGL((gemv_prep_valu_kernel<BPW>), grid, block, s.lds, st, p);
}

hipError_t launch_prep_gemv(const PrepParams& p, const PrepGemvShape& s, hipStream_t st) {
    (void)hipGetLastError();
    if (p.M > 1) {
        const dim3 grid((p.N / 16 + s.spw - 1) / s.spw), block(64 * s.waves);
        if (s.mp == 2) hipLaunchKernelGGL((gemv_prep_rows_kernel<2, 8, 1>), grid, block, s.lds, st, p);
        else if (s.mp == 4 && s.spw == 2) hipLaunchKernelGGL((gemv_prep_rows_kernel<4, 4, 2>), grid, block, s.lds, st, p);
        else if (s.mp == 4) hipLaunchKernelGGL((gemv_prep_rows_kernel<4, 8, 1>), grid, block, s.lds, st, p);
        else hipLaunchKernelGGL((gemv_prep_rows_kernel<8, 8, 1>), grid, block, s.lds, st, p);
        return hipGetLastError();
    }
    switch (s.bpw) {
        case 4: launch_prep_m1_b<4>(p, s, st); break;
        case 8: launch_prep_m1_b<8>(p, s, st); break;
        case 16: launch_prep_m1_b<16>(p, s, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace w4a16
