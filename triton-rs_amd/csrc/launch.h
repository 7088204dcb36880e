// Internal host-side interface between the C-ABI layer (api.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef _Float16 half_t;

// Kernel-internal format id of the prepared layout (prepared.hip), beside the w4a16_format
// values 0..2; never accepted from callers.
constexpr int FMT_PREP = 3;

constexpr int GEMV_MAX_M = 4;        // VALU dot products
constexpr int GEMV_MFMA_MAX_M = 8;   // AWQ with matrix-core dot products

// Split-K counter area: one 32-bit counter per output tile, FLAG_STRIDE words apart (a
// 256-byte line each), in the first SPLITK_FLAG_BYTES of a per-stream workspace; zero
// between calls.
constexpr int FLAG_STRIDE = 64;
constexpr size_t SPLITK_FLAG_BYTES = 2u << 20;
constexpr size_t SPLITK_MAX_TILES = SPLITK_FLAG_BYTES / (FLAG_STRIDE * sizeof(uint32_t));
// Fixed-point split-K hand-off (splitk.h, splitk_fixed_commit): after the counters, one
// 64-bit slot word per output entry, then one 32-bit split mask per entry, all zero between
// calls (room for FIX_MAX_ENTRIES entries). Used when splits <= FIX_MAX_SPLITS and either
// M <= FIX_MAX_M and M * N <= FIX_VALU_MAX_ENTRIES, or the kernel is the row-paired AWQ one
// (M = 3..8) and M * N <= FIX_MAX_ENTRIES. With more entries the atomics cost more than the
// counter protocol's reload: AWQ M = 8, 4096 -> 14336, four splits: 14.5 us with the counter,
// 15.3 us fixed-point on the column-interleaved kernel (whose time also varied with the
// weight data at M = 8, 15.3 to 18.2 us across seeds, so it keeps the counter above M = 4);
// on the row-paired kernel (graph replays, 20 rotated weight sets) M = 5 at N = 14336
// (71,680 entries) 10.84 -> 10.17 us, M = 6 (86,016) 10.94 vs 10.99, M = 8 (114,688)
// 11.27 -> 11.87; at N = 4096 M = 5 / 6 / 8 11.37 / 11.67 / 12.31 -> 10.45 / 11.25 / 12.29.
constexpr int FIX_MAX_SPLITS = 31;
constexpr int FIX_MAX_M = 4;
constexpr size_t FIX_VALU_MAX_ENTRIES = 65536;
constexpr size_t FIX_MAX_ENTRIES = 73728;
constexpr size_t FIX_SLOT_BYTES = FIX_MAX_ENTRIES * (sizeof(uint64_t) + sizeof(uint32_t));

struct GemvParams {
    const half_t* x;          // [M, K] contiguous
    const uint32_t* qweight;  // GPTQ [K/8, N] | AWQ [K, N/8]
    const half_t* scales;     // [K/G, N]
    const uint32_t* qzeros;   // [K/G, N/8] (null for GPTQ_SYM)
    half_t* out;              // [M, N]
    float* ws;                // split-K partials [splits, M, N]
    uint32_t* counters;       // one per column tile (FLAG_STRIDE apart), zero between calls
    uint64_t* slots;          // fixed-point hand-off: one word per output entry, zero between calls
    uint32_t* masks;          // its out-of-range split masks, one per output entry, zero between calls
    int M, N, K, G, zero_offset, splits, col_tiles;
    int fixed;                // 1: fixed-point hand-off (splitk_fixed_commit), 0: counter per tile
};

struct GemvShape {
    bool ok;
    bool mfma;              // AWQ matrix-core kernel (else VALU dot products)
    bool mfma_wide;         // its 8-wave, 1024-row tile (else 4 waves, 256 rows)
    bool awq_rows;          // AWQ matrix-core kernel with row-paired B operands (M >= 3)
    bool gptq_deep;         // GPTQ at M = 1: 8 packed rows per lane (512 k per workgroup)
    bool gptq_narrow;       // GPTQ at M >= 2: 64-column tile (16 lanes per packed row)
    bool awq_deep;          // AWQ VALU kernel at M = 1: 8 waves, 512 rows per workgroup
    bool xcd;               // all splits of a tile on one XCD, hand-off in its L2 (splitk.h)
    int col_tiles, splits, threads;
};

// xcd_placement: the device hands workgroup b to XCD b mod 8 (check_xcd_placement).
// bf16: shapes for bfloat16 elements (no block-diagonal matrix-core GEMV, which is fp16 only)
GemvShape gemv_shape(int fmt, int M, int N, int K, int G, bool xcd_placement, bool bf16 = false);
// bf16: x, scales and out are bfloat16 (the VALU and row-paired AWQ kernels)
hipError_t launch_gemv(int fmt, const GemvParams& p, const GemvShape& s, hipStream_t st, bool bf16 = false);
// Runs a probe kernel on the current device and reports whether workgroups whose ids are
// congruent mod 8 always share an XCD (synchronous; not for use under graph capture).
hipError_t check_xcd_placement(bool* ok);

// Prefill GEMM (large M): dequant-to-LDS MFMA tiles.
struct PrefillParams {
    const half_t* x;
    const uint32_t* qweight;
    const half_t* scales;
    const uint32_t* qzeros;
    half_t* out;
    int M, N, K, G, zero_offset;
    // grouped (fused-MoE) mode only
    const int32_t* sorted_ids;       // [capacity] pair ids, padding = num_pairs
    const int32_t* expert_ids;       // [capacity / block_m]
    const int32_t* num_post_padded;  // device scalar
    int num_pairs, a_div;            // x row of pair p is p / a_div
    int num_experts;                 // expert ids outside [0, num_experts): block skipped
    int64_t qweight_stride, scales_stride, qzeros_stride;   // per expert, in elements
    // expert-tile mode (tiles != nullptr): workgroup row y computes tile y of the list,
    // {first sorted row, rows, expert, 0}, while y < *num_tiles; expert_ids and
    // num_post_padded are then unused
    const int32_t* tiles;
    const int32_t* num_tiles;
    // dense split-K (ksplit > 1): workgroup z computes K stages [z ns, (z+1) ns) into
    // ws[z][M][N] (fp32); the last of a tile's splits sums them in split order
    float* ws;
    uint32_t* counters;       // one per tile (FLAG_STRIDE apart), zero between calls
    int ksplit;
    // gate (nullable): the kernel runs only when *gate == gate_want (a word an earlier kernel
    // on the stream wrote); otherwise every workgroup returns at once
    const uint32_t* gate;
    uint32_t gate_want;
    // expert-tile mode: > 0 selects the XCD-grouped workgroup order over a 1-D grid and is
    // the grid's bound on tiles (set by launch_moe_gemm_tiles)
    int xcd_tiles;
};

struct PrefillShape {
    bool ok;
    bool dma;               // pipelined kernel (LDS-DMA); else the register-staged one
    int bm, bn, col_tiles, row_tiles;
    int ksplit;             // K splits across workgroups (1: none)
    size_t lds;
};

size_t prefill_dma_lds(int bm, int bn);

// max_ksplit caps the K split (1: never split, so no scratch is needed).
PrefillShape prefill_shape(int fmt, int M, int N, int K, int G, int num_cus, int max_ksplit = 8);
// bf16: x, scales and out are bfloat16 (pipelined kernel, dense checkpoint layouts only)
hipError_t launch_prefill(int fmt, const PrefillParams& p, const PrefillShape& s, hipStream_t st,
                          bool bf16 = false);
bool moe_gemm_supported(int N, int K, int G, int block_m);
hipError_t launch_moe_gemm(int fmt, const PrefillParams& p, int block_m, int max_blocks,
                           hipStream_t st);
// Expert-tile grouped GEMM: tile rows tile_bm (128, 192 or 256 with tile columns bn = 256,
// 224 or 128 dividing N; 64 with bn = 256); grid rows max_tiles, the bound of moe_max_tiles.
bool moe_tiles_supported(int N, int K, int G, long long a_rows, int bn);
hipError_t launch_moe_gemm_tiles(int fmt, const PrefillParams& p, int tile_bm, int bn,
                                 int max_tiles, hipStream_t st);

// Fused-MoE helpers (kernels_moe.hip).
hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int renormalize,
                            int32_t* ids, float* weights, hipStream_t st);
hipError_t launch_moe_align(const int32_t* ids, int P, int E, int block_m, int capacity,
                            int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_padded,
                            hipStream_t st, int tile_bm = 0, int32_t* tiles = nullptr,
                            int32_t* num_tiles = nullptr, uint32_t* counters = nullptr,
                            int n_counters = 0);
// Upper bound on the expert tiles of tile_bm rows that P pairs over E experts can need.
inline int moe_max_tiles(int P, int E, int tile_bm) { return (P + tile_bm - 1) / tile_bm + E; }
hipError_t launch_silu_mul(const half_t* gate_up, half_t* out, int inter, int64_t total,
                           hipStream_t st);
hipError_t launch_silu_mul_f32(const float* gate_up, float* out, int inter, int64_t total,
                               hipStream_t st);
hipError_t launch_moe_sum(const half_t* y_pairs, const float* weights, half_t* out, int T,
                          int topk, int K, hipStream_t st);

// Small-batch MFMA GEMM (5 <= M <= 64): waves split K inside a workgroup.
struct SkinnyParams {
    const half_t* x;
    const uint32_t* qweight;
    const half_t* scales;
    const uint32_t* qzeros;
    half_t* out;
    float* ws;
    uint32_t* flags;
    const int32_t* g_idx;   // act-order groups [K], or null
    int M, N, K, G, zero_offset, splits, steps_per_wave, col_tiles;
};

struct SkinnyShape {
    bool ok;
    bool xcd;               // all splits of a tile on one XCD, hand-off in its L2 (splitk.h)
    bool gidx_lds;          // act-order: the workgroup's g_idx slice staged in LDS too
    int bm, cpl, col_tiles, splits, steps_per_wave;
    int waves;              // waves per workgroup
    size_t lds;             // dynamic LDS bytes (act-order group table, g_idx slice)
};

// Largest act-order group table a workgroup stages in LDS.
constexpr size_t SKINNY_GIDX_MAX_LDS = 64 * 1024;

SkinnyShape skinny_shape(int fmt, int M, int N, int K, int G, int num_cus, bool gidx = false,
                         bool xcd_placement = false);
// bf16: x, scales and out are bfloat16
hipError_t launch_skinny(int fmt, const SkinnyParams& p, const SkinnyShape& s, hipStream_t st,
                         bool bf16 = false);

// Generic strided GEMM with the reference kernels' parameter list
// (w4a16_gptq_gemm_typed.rs:110-128, awq_gemm_int4_typed.rs:96-114) plus optional g_idx.
struct StridedParams {
    const half_t* a;
    const uint32_t* qweight;
    const half_t* scales;
    const uint32_t* qzeros;   // null for GPTQ_SYM
    const int32_t* g_idx;     // null: group = k / G
    half_t* c;
    int m, n, k, group_size;
    int stride_am, stride_ak, stride_qwk, stride_qwn, stride_sk, stride_sn;
    int stride_qzk, stride_qzn, stride_cm, stride_cn;
    int zero_offset;
    const uint32_t* gate;     // nullable: run only when *gate == gate_want (as PrefillParams)
    uint32_t gate_want;
};
// bf16: activations, scales and output are bfloat16 (same layouts)
hipError_t launch_strided_gemm(int fmt, const StridedParams& p, hipStream_t st, bool bf16 = false);

// Standalone dequant to a transposed fp16 [N, K] matrix
// (ferrum_dequant_int4.rs:27-139, ferrum_dequant_int4_sym.rs:24-131), and a row-major
// [K, N] variant used by the dense fallback.
struct DequantParams {
    const uint32_t* qweight;
    const half_t* scales;
    const uint32_t* qzeros;
    const int32_t* g_idx;
    half_t* out;
    int K, N, G, zero_offset;
    int transposed;
};
hipError_t launch_dequant(int fmt, const DequantParams& p, hipStream_t st, bool bf16 = false);

// Act-order in group order (act_order.hip): qout = rows of the GPTQ qweight q [K/8, N] taken
// in the order perm (row j of qout = row perm[j] of q); xout [M, K] = x[:, perm].
hipError_t launch_gptq_repack_rows(const uint32_t* q, const int32_t* perm, uint32_t* qout, int K,
                                   int N, hipStream_t st);
// perm (K entries) of the rows in group order, computed on the device from g_idx, and hdr[0]
// (the gate word) = 1 when every group holds exactly G rows, else 0 (perm then the identity).
// hdr[1..3] (16 bytes, zero when first used) and gcopy (K entries) keep what the result was
// computed from, so that a call with the same g_idx, K and G returns after the compare.
// K <= 32768, K / G <= 1024.
hipError_t launch_act_order_perm(const int32_t* g_idx, int32_t* perm, uint32_t* hdr, int32_t* gcopy,
                                 int K, int G, hipStream_t st);
// launch_gptq_repack_rows and launch_gather_columns in one launch (the two passes side by side)
// where K % 32 == 0, K <= 32768 and x, perm, xout are 16-byte aligned; else the two launches.
hipError_t launch_act_order_stage(const uint32_t* q, const int32_t* perm, uint32_t* qout,
                                  const half_t* x, half_t* xout, int M, int K, int N,
                                  hipStream_t st);
hipError_t launch_gather_columns(const half_t* x, const int32_t* perm, half_t* xout, int M, int K,
                                 hipStream_t st);

// Prepared layout (prepared.hip): strips of 16 columns, each one contiguous run of
// prep_strip_bytes(K, G) bytes: the strip's table (per block of 128 rows, R = max(1, 128/G)
// rows of 16 entries, fp16 scale | zero point << 16; padded to 256 bytes), then K / 128 blocks
// of 1 KiB. Needs N % 16 == 0, K % 128 == 0, K % G == 0 and G one of 32, 64 or a multiple
// of 128.
constexpr bool prep_group_ok(int G) { return G == 32 || G == 64 || (G >= 128 && G % 128 == 0); }
constexpr int prep_table_rows(int G) { return G < 128 ? 128 / G : 1; }   // per block
constexpr uint32_t prep_table_words(int K, int G) {
    return (uint32_t)(((K / 128) * prep_table_rows(G) * 16 + 63) & ~63);
}
constexpr size_t prep_strip_bytes(int K, int G) { return (size_t)K * 8 + (size_t)prep_table_words(K, G) * 4; }
inline size_t prep_total_bytes(int K, int N, int G) { return (size_t)(N / 16) * prep_strip_bytes(K, G); }
constexpr int PREP_MAX_K = 32768;

struct PrepParams {
    const half_t* x;              // [M, K]
    const unsigned char* prep;    // prepared weights
    half_t* out;                  // [M, N]
    int M, N, K, G;
    uint32_t strip_bytes;
};
struct PrepGemvShape {
    bool ok;
    int bpw;      // blocks (128 rows x 16 columns) per wave, at most
    int waves;    // waves per workgroup (one workgroup per strip)
    bool mfma;    // matrix-core dot products (group_size % 128 == 0), else VALU dot2
    int mp;       // M > 1: rows per block slot of the A operand (2, 4 or 8)
    int spw;      // M > 1: strips per workgroup
    size_t lds;   // dynamic LDS bytes
};
constexpr int PREP_GEMV_MAX_M = 8;
// M <= 64 on the prepared layout (G % 128 == 0) with the activations in MFMA fragment order
// (prepared.hip): one workgroup per S strips, its waves over K.
struct PrepFragParams {
    const half_t* x;              // x [M, K], row-major
    // checkpoint source (launch_ck_frag): GPTQ qweight [K/8, N], scales [K/G, N], qzeros
    // [K/G, N/8] (GPTQ_SYM: unused), zero = nibble + zero_offset
    const uint32_t* qweight;
    const half_t* scales;
    const uint32_t* qzeros;
    int zero_offset;
    const int32_t* g_idx;         // checkpoint, act-order (nullable): each row's group
    const unsigned char* prep;    // prepared weights (fewer than 2^31 bytes)
    half_t* out;                  // [M, N]
    int M, N, K, G;
    uint32_t strip_bytes;
};
struct PrepFragShape {
    bool ok;
    int mt;       // 16-row tiles of x
    int s;        // strips per workgroup
    int bpw;      // blocks per wave
    int pd;       // blocks of loads in flight per wave
    int waves;    // per workgroup
    size_t lds;   // dynamic LDS bytes
};
constexpr int PREP_FRAG_MAX_M = 64;
hipError_t launch_prepare_layout(int fmt, const uint32_t* qweight, const half_t* scales,
                                 const uint32_t* qzeros, void* out, int K, int N, int G,
                                 int zero_offset, hipStream_t st);
hipError_t launch_prep_dequant(const void* prep, half_t* out, int K, int N, int G, int transposed,
                               hipStream_t st);
PrepGemvShape prep_gemv_shape(int M, int N, int K, int G);
hipError_t launch_prep_gemv(const PrepParams& p, const PrepGemvShape& s, hipStream_t st);
// act: rows in the checkpoint's own order with p.g_idx (any group size of the layout,
// K <= 4096, a table of at most 4096 entries)
PrepFragShape prep_frag_shape(int M, int N, int K, int G, bool act = false);
hipError_t launch_prep_frag(const PrepFragParams& p, const PrepFragShape& s, hipStream_t st);
// The small-batch kernel on a GPTQ / GPTQ_SYM checkpoint as stored (no split-K, no scratch);
// act: with g_idx (any group size, K <= 4096, a table of at most 4096 entries)
PrepFragShape ck_frag_shape(int fmt, int M, int N, int K, int G, bool act = false);
hipError_t launch_ck_frag(int fmt, const PrepFragParams& p, const PrepFragShape& s, hipStream_t st);

// ------------------------------------------------------------------ op layer (api.cpp)

// Split-K scratch of one call: tile counters (FLAG_STRIDE apart), the fixed-point hand-off's
// slot words and split masks (FIX_MAX_ENTRIES each), fp32 partials. Counters, slots and masks
// are zero between calls.
struct Scratch {
    uint32_t* counters;
    uint64_t* slots;
    uint32_t* masks;
    float* partials;
};
// Where a call's scratch comes from: the per-stream workspace the library allocates (grows on
// demand), or a fixed area (limits below; get() never allocates).
struct ScratchSource {
    size_t max_partial_bytes;
    size_t max_tiles;
    bool may_probe;   // may run the XCD placement probe (it allocates)
    bool may_allocate;   // may take per-stream buffers (act-order repack beyond 64 rows)
    int (*get)(hipStream_t st, size_t partial_bytes, Scratch* out);
};
ScratchSource alloc_scratch_source();

// w4a16_gemm with the scratch taken from `src`.
int gemm_impl(void* stream, int fmt, const void* x, const void* qweight, const void* scales,
              const void* qzeros, const int32_t* g_idx, void* out, int32_t M, int32_t N,
              int32_t K, int32_t G, int32_t zero_offset, const ScratchSource& src);
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);

// Allocation-free entry point's per-device set-up (noalloc.hip): looks up the device's copy of
// the scratch array and clears it (on `st`; waited for when st is the null stream).
int noalloc_setup(hipStream_t st = nullptr);

}  // namespace w4a16
