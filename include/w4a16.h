/*
 * w4a16.h -- C ABI of the MI355X (gfx950) W4A16 library: int4 weight-only GEMM for the
 * GPTQ and AWQ packings, its act-order (g_idx) and fused-MoE variants, and a HIP runtime
 * that stands in for the reference's DeviceRuntime trait.
 *
 * Replaces, for this path, what the reference compiles through Triton and launches with
 * cudarc (sizzlecar/triton-rs):
 *   crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:103-129  (GPTQ GEMM parameter list)
 *   crates/triton-dsl/examples/awq_gemm_int4_typed.rs:94-115     (AWQ GEMM parameter list)
 *   crates/triton-dsl/examples/ferrum_dequant_int4.rs:27-37      (GPTQ asym dequant)
 *   crates/triton-dsl/examples/ferrum_dequant_int4_sym.rs:24-31  (GPTQ sym dequant)
 *   crates/triton-runtime/src/lib.rs:18-85                       (RuntimeError, KernelArg,
 *                                                                 DeviceRuntime)
 *
 * Conventions (all functions):
 *  - Return int status: 0 (W4A16_OK) or a w4a16_status error. Nothing throws or aborts.
 *    w4a16_last_error() returns the calling thread's message for its last failure.
 *  - Arguments are validated on the host before any HIP call, so every argument error is
 *    reported without touching the GPU.
 *  - Pointers are device pointers (hipMalloc'd or HIP-visible); fp16 data is IEEE binary16.
 *  - `stream` is a hipStream_t (NULL = the null stream). Work is enqueued asynchronously.
 *  - Matrices are row-major. Sizes and strides are int32, as in the reference (its offsets
 *    are i32, w4a16_gptq_gemm_typed.rs:119-128); offsets are computed in 64 bits here.
 */
#ifndef W4A16_H
#define W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_API __attribute__((visibility("default")))

/* Status codes. ModuleLoad / InvalidLaunchConfig / Device / BackendDisabled mirror the
 * reference's RuntimeError variants (crates/triton-runtime/src/lib.rs:18-35). */
typedef enum {
    W4A16_OK = 0,
    W4A16_ERR_INVALID_ARG = 1,       /* null pointer, bad size, bad divisibility, bad handle */
    W4A16_ERR_UNSUPPORTED = 2,       /* valid request outside what this build implements */
    W4A16_ERR_DEVICE = 3,            /* RuntimeError::Device: a HIP call failed */
    W4A16_ERR_MODULE_LOAD = 4,       /* RuntimeError::ModuleLoad */
    W4A16_ERR_LAUNCH_CONFIG = 5,     /* RuntimeError::InvalidLaunchConfig */
    W4A16_ERR_BACKEND_DISABLED = 6,  /* RuntimeError::BackendDisabled: no usable HIP device */
    W4A16_ERR_NOT_FOUND = 7          /* kernel name not present in a loaded module */
} w4a16_status;

/* Weight packings.
 *  GPTQ     qweight int32 [K/8, N], row k in nibble slot k%8 (w4a16_gptq_gemm_typed.rs:15-32);
 *           qzeros int32 [K/G, N/8], column n in slot n%8, zero = nibble + zero_offset
 *           (the reference GEMM uses +1, :224-236; its asym dequant uses 0).
 *  GPTQ_SYM as GPTQ with zero = 8 and no qzeros (ferrum_dequant_int4_sym.rs:60).
 *  AWQ      qweight int32 [K, N/8] and qzeros int32 [K/G, N/8]; column n in slot
 *           (n%8)/2 + (n%8)%2*4, i.e. [0,4,1,5,2,6,3,7]; zero = nibble
 *           (awq_gemm_int4_typed.rs:10-31, 139-151, 203-205).
 * scales are fp16 [K/G, N] for all three. */
typedef enum { W4A16_FMT_GPTQ = 0, W4A16_FMT_GPTQ_SYM = 1, W4A16_FMT_AWQ = 2 } w4a16_format;

/* OR-ed into `fmt` of w4a16_gemm, w4a16_gemm_noalloc, w4a16_gemm_plan and w4a16_dequant:
 * x, scales and out are bfloat16 instead of fp16 (the reference kernels are generic over the
 * element type, w4a16_gptq_gemm_typed.rs:65-67, and name bf16; its v0 instantiates f16).
 * A weight dequantises to RNE_bf16(f32(q - z) * f32(s)), products accumulate in fp32 and the
 * output is rounded to bf16 once. Plain group order runs the same kernels as fp16 (the
 * GEMVs, the small-batch kernel up to 64 rows, the pipelined prefill beyond; bf16 MFMA and
 * v_dot2c_f32_bf16) except the block-diagonal AWQ GEMV (GPTQ at 5..8 rows takes the
 * small-batch kernel); w4a16_gemm_plan reports which; act-order runs as for fp16. Shapes
 * those kernels reject run the generic kernel. The other entry points reject
 * the flag as an unknown format. */
#define W4A16_BF16 0x100

/* Kernel regimes reported by w4a16_gemm_plan(). */
typedef enum {
    W4A16_KERNEL_GEMV = 1,       /* decode: split-K GEMV, VALU dot2, no MFMA */
    W4A16_KERNEL_SKINNY = 2,     /* small batch: MFMA, weights streamed once */
    W4A16_KERNEL_PREFILL = 3,    /* large M: dequant-to-LDS + MFMA tiles */
    W4A16_KERNEL_STRIDED = 4     /* generic strided kernel (any layout, any shape) */
} w4a16_kernel;

W4A16_API const char* w4a16_last_error(void);
W4A16_API const char* w4a16_version(void);

/* Optional set-up for `device` (it is current again on return): caches the device's CU
 * count and runs the workgroup-placement probe the decode kernels' L2-local split-K hand-off
 * depends on. Without it both happen on the first call; a first call made while its stream
 * is being captured into a HIP graph cannot probe (probing synchronises) and uses the
 * device-scope hand-off instead. No reference counterpart. */
W4A16_API int w4a16_init(int32_t device);

/* ------------------------------------------------------------------ op level */

/* out[M, N] = x[M, K] @ W16[K, N], W16 = RNE_f16((q - z) * scale[g, n]) with
 * g = g_idx ? g_idx[k] : k / group_size; fp32 accumulation; fp16 output.
 * Contiguous row-major tensors. qzeros is ignored (may be NULL) for GPTQ_SYM. g_idx
 * (int32 [K], values in [0, K/group_size); values outside are clamped into it) is optional
 * and, in the reference, absent: it adds GPTQ act-order. Requirements: M, N, K, group_size >= 1; K % group_size == 0;
 * N % 8 == 0; K % 8 == 0 for GPTQ formats. The kernel is chosen by shape (see
 * w4a16_gemm_plan). The split-K kernels use a per-(device, stream) workspace that the
 * library allocates on first use of a size; a larger size later allocates a new one and
 * retires the old one without freeing it (HIP graphs captured earlier keep using it), so a
 * captured call stays valid for the life of the process. Growing the workspace is not
 * possible under stream capture: make one call of the largest size before capturing, or
 * the call fails with W4A16_ERR_UNSUPPORTED. Concurrent calls on different streams are
 * safe. With g_idx from 65 to 128 rows (GPTQ formats, K <= 4096) the small-batch kernel runs
 * in two row chunks; beyond that (K <= 32768, K / group_size <= 1024) each
 * call also computes the group order of the rows on the device, repacks the rows and gathers
 * x into per-(device, stream) buffers (grown like the workspace) and runs the prefill
 * kernel on them; when g_idx's groups do not each hold exactly group_size rows (or an entry
 * is out of range) the generic kernel runs instead, decided on the device. */
W4A16_API int w4a16_gemm(void* stream, int fmt, const void* x, const void* qweight,
                         const void* scales, const void* qzeros, const int32_t* g_idx,
                         void* out, int32_t M, int32_t N, int32_t K, int32_t group_size,
                         int32_t gptq_zero_offset);

/* No counterpart in the reference: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and
 * results as w4a16_gemm, but the split-K scratch (counters, fixed-point hand-off slots,
 * fp32 partials) lives in a fixed device array of w4a16_gemm_noalloc_scratch_bytes() bytes
 * (8 MiB: at most 1024 split-K tiles and 6.9 MiB of partials), one per device, held until the
 * process ends; the call itself allocates nothing. A call whose planned kernel would need
 * more than that runs the prefill kernel with the largest K split whose partials fit (down
 * to none, which needs no scratch), or the generic kernel, and act-order beyond the
 * small-batch kernel's rows (and its row chunks) runs the generic kernel (the
 * repacked rows would not fit), so such results may differ from w4a16_gemm's in the last bits.
 * All calls on one device share its array: calls that overlap in time on one device (other
 * streams or threads) race and must be serialised by the caller. The device's array is set
 * up by w4a16_init (recommended before capture) or by the first call on the device. */
W4A16_API int w4a16_gemm_noalloc(void* stream, int fmt, const void* x, const void* qweight,
                                 const void* scales, const void* qzeros, const int32_t* g_idx,
                                 void* out, int32_t M, int32_t N, int32_t K, int32_t group_size,
                                 int32_t gptq_zero_offset);
W4A16_API size_t w4a16_gemm_noalloc_scratch_bytes(void);

/* GPTQ act-order (desc_act) in group order; no reference counterpart (the reference has no
 * act-order, w4a16_gptq_gemm_typed.rs:221 uses group k / group_size).
 * w4a16_prepare_act_order, once per checkpoint: perm_out (int32 [K]) = the rows sorted by
 * g_idx, stable in k; qweight_out (GPTQ qweight [K/8, N], not aliasing qweight) = the rows of
 * qweight in that order. Every group must hold exactly group_size rows (a desc_act
 * checkpoint's g_idx is a permutation of repeat(0 .. K/G-1, G)); g_idx is read on the host,
 * so the call synchronises `stream` and cannot be captured. scales and qzeros are unchanged.
 * w4a16_gemm_act_order then computes the act-order product x @ W16 from the prepared weights
 * as x[:, perm] @ W16' with plain group order: a gather of x's columns (into a per-(device,
 * stream) buffer the library keeps, growing as w4a16_gemm's workspace does), then the kernel
 * w4a16_gemm plans for (M, N, K) without g_idx (GEMV, small batch or prefill). */
W4A16_API int w4a16_prepare_act_order(void* stream, int fmt, const void* qweight,
                                      const int32_t* g_idx, int32_t K, int32_t N,
                                      int32_t group_size, void* qweight_out, int32_t* perm_out);
W4A16_API int w4a16_gemm_act_order(void* stream, int fmt, const void* x, const void* qweight,
                                   const void* scales, const void* qzeros, const int32_t* perm,
                                   void* out, int32_t M, int32_t N, int32_t K, int32_t group_size,
                                   int32_t gptq_zero_offset);

/* Prepared (kernel-native) layout: the one-time checkpoint repack behind the same op API.
 * Replaces nothing in the reference kernels, which read the checkpoint as stored; it is the
 * load-time step of the loader that feeds them (w4a16_gptq_gemm_typed.rs:11-13, :55-60:
 * ferrum's loader ships qweight, scales and qzeros; awq_gemm_int4_typed.rs:26-31: the AWQ
 * packing), done once so that every later call streams the weights in the order the
 * kernels consume them.
 * Layout: strips of 16 columns, strip s one contiguous run of bytes: first the strip's table,
 * per block of 128 rows R = max(1, 128 / group_size) rows of 16 32-bit entries (entry c of a
 * row: the group's fp16 scale for column 16 s + c in bits 0..15, its full zero point in bits
 * 16..31: the GPTQ nibble + gptq_zero_offset, 8 for GPTQ_SYM, the AWQ nibble), padded to 256
 * bytes; then K/128 blocks of 1 KiB (block kb: 64 lanes x 16 bytes, lane l = column
 * 16 s + l % 16, rows 128 kb + 32 (l / 16) + [0, 32) as four words of 8 rows; row i of a word
 * in nibble slot (i >> 1) | ((i & 1) << 2)). Any of the three formats gives the same layout
 * for the same weights W16 = RNE_f16((q - z) * s).
 * Shapes: N % 16 == 0, K % 128 == 0, group_size 32, 64 or a multiple of 128,
 * K % group_size == 0, K <= 32768.
 *
 * w4a16_prepared_bytes: size of the prepared buffer (0 when the shape is not supported).
 * w4a16_prepare_layout: writes it (256-byte aligned `prepared`, not overlapping the inputs);
 *   asynchronous on `stream`, no host synchronisation, no allocation.
 * w4a16_gemm_prepared: out[M, N] = x[M, K] @ W16 from prepared weights. perm (nullable):
 *   for an act-order checkpoint first repacked by w4a16_prepare_act_order, the permutation it
 *   returned; x's columns are then gathered by it first (as w4a16_gemm_act_order does, into a
 *   per-(device, stream) buffer the library keeps). M = 1 runs a GEMV with one workgroup per
 *   strip over all of K (no split-K, no scratch). With group_size a multiple of 128, 5..64 rows
 *   (4 where K <= 4096; 2..64 with perm) run a small-batch kernel, one workgroup per 1, 2 or
 *   4 strips over all of K (no split-K), which reads x (gathered by perm) as stored and puts
 *   it in the matrix cores' operand order itself.
 * w4a16_dequant_prepared: W16 as fp16 [K, N] (transposed = 0) or [N, K] (= 1), bit-exact. */
W4A16_API size_t w4a16_prepared_bytes(int32_t K, int32_t N, int32_t group_size);
W4A16_API int w4a16_prepare_layout(void* stream, int fmt, const void* qweight, const void* scales,
                                   const void* qzeros, int32_t K, int32_t N, int32_t group_size,
                                   int32_t gptq_zero_offset, void* prepared,
                                   size_t prepared_bytes);
W4A16_API int w4a16_gemm_prepared(void* stream, const void* x, const void* prepared,
                                  const int32_t* perm, void* out, int32_t M, int32_t N,
                                  int32_t K, int32_t group_size);
W4A16_API int w4a16_dequant_prepared(void* stream, const void* prepared, void* out, int32_t K,
                                     int32_t N, int32_t group_size, int transposed);
/* w4a16_gemm_prepared_gidx: out[M, N] = x[M, K] @ W16 for an act-order (desc_act) GPTQ
 * checkpoint prepared as stored (w4a16_prepare_layout on its qweight, scales and qzeros, rows
 * in their own order): g_idx [K] gives row k's group, read from the strips' tables (their
 * rows hold every group's scale and zero point). No counterpart in the reference, whose GEMM
 * takes group k / group_size (w4a16_gptq_gemm_typed.rs:221); it spares an act-order layer the
 * group-order repack (w4a16_prepare_act_order) and the per-call gather of x's columns. Up to
 * 64 rows with K <= 4096 a small-batch kernel reading x as stored, one workgroup per 1, 2 or
 * 4 strips over all of K; other shapes the generic kernel. g_idx entries outside
 * [0, K / group_size) are clamped. Same alignment as w4a16_gemm_prepared, g_idx 16-byte
 * aligned. */
W4A16_API int w4a16_gemm_prepared_gidx(void* stream, const void* x, const void* prepared,
                                       const int32_t* g_idx, void* out, int32_t M, int32_t N,
                                       int32_t K, int32_t group_size);

/* Which kernel w4a16_gemm would run for this problem (no GPU access). */
W4A16_API int w4a16_gemm_plan(int fmt, int32_t M, int32_t N, int32_t K, int32_t group_size,
                              int has_g_idx, int* kernel);

/* ------------------------------------------------------------------ kernel level
 * The reference kernels' exact parameter lists (a_ptr, qweight_ptr, scales_ptr, qzeros_ptr,
 * c_ptr, m, n, k, group_size, 10 strides), prefixed by the stream. Any strides (in
 * elements of the tensor's own type), any M/N/K; masked tails read as zero. */

/* Dense row-major operands (stride_ak = stride_qwn = stride_sn = stride_qzn = stride_cn = 1,
 * stride_am = k, stride_qwk = n (GPTQ) or n / 8 (AWQ), stride_sk = n, stride_qzk = n / 8,
 * stride_cm = n; 16-byte aligned pointers; k % group_size == 0, n % 8 == 0) go to the
 * kernels w4a16_gemm plans; other layouts run the generic strided kernel.
 * w4a16_typed_plan reports which, without touching the GPU (aligned16: whether every
 * pointer will be 16-byte aligned). */
W4A16_API int w4a16_typed_plan(int fmt, int32_t m, int32_t n, int32_t k, int32_t group_size,
                               const int32_t* strides10, int aligned16, int* kernel);

/* replaces w4a16_gptq_gemm_typed (w4a16_gptq_gemm_typed.rs:103-129), zero = nibble + 1 */
W4A16_API int w4a16_gptq_gemm_typed(void* stream, const void* a_ptr, const void* qweight_ptr,
                                    const void* scales_ptr, const void* qzeros_ptr,
                                    void* c_ptr, int32_t m_size, int32_t n_size,
                                    int32_t k_size, int32_t group_size, int32_t stride_am,
                                    int32_t stride_ak, int32_t stride_qwk, int32_t stride_qwn,
                                    int32_t stride_sk, int32_t stride_sn, int32_t stride_qzk,
                                    int32_t stride_qzn, int32_t stride_cm, int32_t stride_cn);

/* replaces awq_gemm_int4_typed (awq_gemm_int4_typed.rs:94-115) */
W4A16_API int awq_gemm_int4_typed(void* stream, const void* a_ptr, const void* qweight_ptr,
                                  const void* scales_ptr, const void* qzeros_ptr, void* c_ptr,
                                  int32_t m_size, int32_t n_size, int32_t k_size,
                                  int32_t group_size, int32_t stride_am, int32_t stride_ak,
                                  int32_t stride_qwk, int32_t stride_qwn, int32_t stride_sk,
                                  int32_t stride_sn, int32_t stride_qzk, int32_t stride_qzn,
                                  int32_t stride_cm, int32_t stride_cn);

/* replaces dequant_int4_to_fp16 (ferrum_dequant_int4.rs:27-37): GPTQ qweight [K/8, N],
 * qzeros [K/G, N/8] with zero = nibble (no +1), output fp16 TRANSPOSED [N, K]
 * (out[n*K + k]). n_div_8 must equal n_dim / 8. */
W4A16_API int dequant_int4_to_fp16(void* stream, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, void* output, int32_t k_dim,
                                   int32_t n_dim, int32_t group_size, int32_t n_div_8);

/* replaces dequant_int4_sym_to_fp16 (ferrum_dequant_int4_sym.rs:24-31): zero = 8. */
W4A16_API int dequant_int4_sym_to_fp16(void* stream, const int32_t* qweight, const void* scales,
                                       void* output, int32_t k_dim, int32_t n_dim,
                                       int32_t group_size);

/* Dequantise any format to fp16, row-major [K, N] (transposed = 0) or [N, K] (= 1).
 * g_idx optional. No reference counterpart beyond the two functions above. */
W4A16_API int w4a16_dequant(void* stream, int fmt, const void* qweight, const void* scales,
                            const void* qzeros, const int32_t* g_idx, void* out, int32_t K,
                            int32_t N, int32_t group_size, int32_t gptq_zero_offset,
                            int transposed);

/* ------------------------------------------------------------------ fused MoE
 * Not in the reference (it has no MoE kernel; the benchmark's Mixtral-like layer needs one). The
 * pieces compose as: route -> align -> grouped GEMM (w1|w3) -> silu*mul -> grouped GEMM (w2)
 * -> weighted sum. Pairs are (token t, slot j) with index p = t * topk + j, P = T * topk. */

/* softmax over E fp32 logits per token, top-k (ties -> lower expert index); weights are the
 * chosen probabilities, renormalised to sum to 1 when `renormalize` != 0.
 * topk_ids int32 [T, topk], topk_weights fp32 [T, topk]. E <= 256, topk <= 8. */
W4A16_API int w4a16_moe_route(void* stream, const float* logits, int32_t T, int32_t E,
                              int32_t topk, int32_t renormalize, int32_t* topk_ids,
                              float* topk_weights);

/* Sort pairs by expert (stable in p), padding each expert to a multiple of block_m with the
 * sentinel num_pairs. sorted_ids int32 [capacity], expert_ids int32 [capacity / block_m],
 * *num_tokens_post_padded = padded length (device). capacity must be a multiple of block_m
 * and >= num_pairs + E * (block_m - 1). topk_ids are read on the device: a pair whose id is
 * outside [0, E) is dropped (it appears in no block, so a grouped GEMM leaves its output row
 * unwritten). */
W4A16_API int w4a16_moe_align(void* stream, const int32_t* topk_ids, int32_t num_pairs, int32_t E,
                              int32_t block_m, int32_t capacity, int32_t* sorted_ids,
                              int32_t* expert_ids, int32_t* num_tokens_post_padded);

/* Grouped W4A16 GEMM over expert-sorted blocks: for every block of block_m sorted pairs with
 * expert e, out[p, :] = a[p / a_div, :] @ W16_e, W16_e from the e-th slice of the stacked
 * qweight / scales / qzeros (expert strides in elements; num_experts slices). out is
 * [num_pairs, N]; padding rows are skipped. N % 256 == 0, K % 64 == 0, block_m in {64, 128}.
 * The routing tables are read on the device: a block whose expert id is outside
 * [0, num_experts) is skipped, and a sorted id outside [0, num_pairs) is padding. */
W4A16_API int w4a16_moe_gemm(void* stream, int fmt, const void* a, int32_t a_div,
                             const void* qweight, const void* scales, const void* qzeros,
                             int64_t qweight_expert_stride, int64_t scales_expert_stride,
                             int64_t qzeros_expert_stride, int32_t num_experts,
                             const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                             void* out, int32_t num_pairs, int32_t N, int32_t K,
                             int32_t group_size, int32_t block_m, int32_t capacity,
                             int32_t gptq_zero_offset);

/* replaces fused_silu_mul_interleaved_f16 (crates/triton-kernels/src/elementwise.rs:188-212):
 * out[idx] = f16(silu(g) * u) for idx < total, b = idx / inter, i = idx % inter,
 * g = gate_up[b * 2 * inter + i], u = gate_up[b * 2 * inter + inter + i],
 * silu(g) = g / (1 + exp(-g)) in f32. Any inter >= 1 and total >= 0 (normally batch * inter). */
W4A16_API int fused_silu_mul_interleaved_f16(void* stream, const void* gate_up, void* out,
                                             int32_t inter, int32_t total);

/* replaces fused_silu_mul_interleaved_f32 (crates/triton-kernels/src/elementwise.rs:214-250):
 * the same indexing over f32 buffers, out[idx] = silu(g) * u in f32. Same argument rules. */
W4A16_API int fused_silu_mul_interleaved_f32(void* stream, const float* gate_up, float* out,
                                             int32_t inter, int32_t total);

/* out[t, :] = f16(sum_j topk_weights[t, j] * f32 y_pairs[t * topk + j, :]); K % 8 == 0. */
W4A16_API int w4a16_moe_sum(void* stream, const void* y_pairs, const float* topk_weights,
                            void* out, int32_t T, int32_t topk, int32_t K);

/* Bytes of workspace w4a16_fused_moe needs (routing tables, expert tile list, fp16
 * intermediates and, when I >= 8192, the down projection's fp32 split-K partials). */
W4A16_API size_t w4a16_fused_moe_workspace_size(int32_t T, int32_t E, int32_t topk, int32_t I,
                                                int32_t K, int32_t block_m);

/* Whole MoE layer: y[T, K] from x[T, K] and router logits[T, E]. Expert weights are stacked
 * along a leading expert dimension in the chosen packing: w13 is [E] x (K -> 2I) with columns
 * [0, I) = w1 (gate) and [I, 2I) = w3 (up); w2 is [E] x (I -> K). `workspace` (256-byte
 * aligned, w4a16_fused_moe_workspace_size bytes) is caller-owned. */
W4A16_API int w4a16_fused_moe(void* stream, int fmt, const void* x, const float* router_logits,
                              int32_t T, int32_t K, int32_t I, int32_t E, int32_t topk,
                              int32_t renormalize, const void* w13_qweight, const void* w13_scales,
                              const void* w13_qzeros, const void* w2_qweight,
                              const void* w2_scales, const void* w2_qzeros, int32_t group_size,
                              int32_t block_m, int32_t gptq_zero_offset, void* workspace,
                              size_t workspace_bytes, void* out);

/* The same layer on expert weights in the prepared layout (no reference counterpart, like
 * w4a16_prepare_layout): w13_prepared holds E consecutive w4a16_prepare_layout outputs of the
 * experts' K -> 2I matrices, each w4a16_prepared_bytes(K, 2I, group_size) bytes (256-byte
 * aligned), w2_prepared E of the I -> K matrices. Same routing, tiles and workspace as
 * w4a16_fused_moe (w4a16_fused_moe_workspace_size); the grouped GEMMs read the prepared strips.
 * Needs group_size % 64 == 0 and the shapes the expert-tile kernels take (else
 * W4A16_ERR_UNSUPPORTED). */
W4A16_API int w4a16_fused_moe_prepared(void* stream, const void* x, const float* router_logits,
                                       int32_t T, int32_t K, int32_t I, int32_t E, int32_t topk,
                                       int32_t renormalize, const void* w13_prepared,
                                       const void* w2_prepared, int32_t group_size,
                                       int32_t block_m, void* workspace, size_t workspace_bytes,
                                       void* out);

/* ------------------------------------------------------------------ runtime
 * A HIP backend for the reference's DeviceRuntime trait (crates/triton-runtime/src/
 * lib.rs:64-85): load a code object, launch a kernel by name with KernelArg-style
 * arguments. Plus the allocation / copy / stream / event calls the reference's examples
 * take from cudarc (crates/triton-runtime/examples/run_vec_add.rs:70-123). */

typedef struct hiprt_ctx hiprt_ctx;
typedef struct hiprt_module hiprt_module;

/* KernelArg (crates/triton-runtime/src/lib.rs:46-60) as a tagged union. */
typedef enum {
    HIPRT_ARG_I32 = 0,
    HIPRT_ARG_U32 = 1,
    HIPRT_ARG_I64 = 2,
    HIPRT_ARG_F32 = 3,
    HIPRT_ARG_DEVICE_PTR = 4,
    HIPRT_ARG_BYTES = 5
} hiprt_arg_kind;

typedef struct {
    int32_t kind;           /* hiprt_arg_kind */
    uint32_t size;          /* HIPRT_ARG_BYTES only: byte count */
    union {
        int32_t i32;
        uint32_t u32;
        int64_t i64;
        float f32;
        uint64_t device_ptr;
        const void* bytes;  /* copied into the kernel parameter buffer, 8-byte aligned */
    } v;
} hiprt_arg;

/* Bind a context to a device (fails with BACKEND_DISABLED when there is none). */
W4A16_API int hiprt_create(int32_t device, hiprt_ctx** out);
W4A16_API int hiprt_destroy(hiprt_ctx* ctx);

/* DeviceRuntime::load_module: `binary` is a gfx950 code object (.hsaco); it is borrowed. */
W4A16_API int hiprt_module_load(hiprt_ctx* ctx, const void* binary, size_t size,
                                hiprt_module** out);
W4A16_API int hiprt_module_unload(hiprt_module* module);

/* DeviceRuntime::launch. Arguments are packed at their natural alignment. A launch of
 * w4a16_gptq_gemm_typed or awq_gemm_int4_typed from the library's own w4a16_typed.hsaco
 * (recognised at load by its marker symbol) that follows that module's contract (the 19
 * arguments, optionally the two scratch pointers; grid (cdiv(m, 64), cdiv(n, 64), 1), block
 * (256, 1, 1), no dynamic LDS) is run by the C-ABI entry of the same name, i.e. on the planned
 * kernels; any other launch runs the named kernel of the module as given. */
W4A16_API int hiprt_launch(hiprt_ctx* ctx, const hiprt_module* module, const char* kernel_name,
                           const uint32_t grid[3], const uint32_t block[3],
                           uint32_t shared_mem_bytes, void* stream, const hiprt_arg* args,
                           size_t nargs);

W4A16_API int hiprt_stream_create(hiprt_ctx* ctx, void** stream);
W4A16_API int hiprt_stream_destroy(void* stream);
W4A16_API int hiprt_stream_synchronize(void* stream);
W4A16_API int hiprt_malloc(hiprt_ctx* ctx, size_t bytes, uint64_t* device_ptr);
W4A16_API int hiprt_free(hiprt_ctx* ctx, uint64_t device_ptr);
W4A16_API int hiprt_memcpy_htod_async(uint64_t dst, const void* src, size_t bytes, void* stream);
W4A16_API int hiprt_memcpy_dtoh_async(void* dst, uint64_t src, size_t bytes, void* stream);
W4A16_API int hiprt_memset_async(uint64_t dst, int value, size_t bytes, void* stream);
W4A16_API int hiprt_event_create(void** event);
W4A16_API int hiprt_event_destroy(void* event);
W4A16_API int hiprt_event_record(void* event, void* stream);
W4A16_API int hiprt_event_synchronize(void* event);
W4A16_API int hiprt_event_elapsed_ms(void* start, void* stop, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* W4A16_H */
