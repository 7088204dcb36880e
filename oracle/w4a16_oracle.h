/*
 * CPU oracle for the W4A16 (int4 weight x fp16 activation) path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker.
 * The product path (the HIP library under triton-rs_amd/) never links it.
 *
 * This is a plain-C restatement of the reference's arithmetic for the path.
 * The reference is Rust DSL source that cannot be compiled here (no cargo, no
 * CUDA), so there is no oracle/_ref build; every function below cites the
 * reference file:line it follows and the check that pins it (tests/test_oracle*.py).
 *
 * All fp16 values are passed as their IEEE-754 binary16 bit patterns (uint16_t).
 */
#ifndef W4A16_ORACLE_H
#define W4A16_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight formats. Same numbering as include/w4a16.h. */
enum { ORC_FMT_GPTQ = 0, ORC_FMT_GPTQ_SYM = 1, ORC_FMT_AWQ = 2 };

/* binary16 <-> binary32, round-to-nearest-even, hand-written from the
 * IEEE-754 bit layout. Mirrors MLIR arith.truncf / arith.extf
 * (crates/triton-ir/src/module.rs:726-731). */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* bfloat16 (bit patterns): f32 -> bf16 round to nearest even (NaN kept), bf16 -> f32 exact. */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);
void orc_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void orc_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* Nibble slot that column n occupies inside an AWQ word:
 * (n%8)/2 + (n%8)%2*4 (crates/triton-dsl/examples/awq_gemm_int4_typed.rs:139-151). */
int orc_awq_slot(int n);

/* Nibble `slot` (0..7) of a packed int32, logical shift then & 0xF
 * (arith.shrui, crates/triton-ir/src/dialect/arith.rs:171). */
int orc_nibble(int32_t word, int slot);

/* Integer weight q[k,n] (0..15) of a packed qweight.
 *   GPTQ / GPTQ_SYM: qweight [K/8, N], slot k%8  (w4a16_gptq_gemm_typed.rs:175-180, 213-217)
 *   AWQ:             qweight [K, N/8], slot awq  (awq_gemm_int4_typed.rs:139-151, 189-195) */
int orc_qweight_at(int fmt, const int32_t* qweight, int K, int N, int k, int n);

/* Zero point of (group g, column n).
 *   GPTQ:     nibble(qzeros[g, n/8], n%8) + zero_offset   (w4a16_gptq_gemm_typed.rs:231-236,
 *             offset 1; ferrum_dequant_int4.rs:67-76 uses offset 0)
 *   GPTQ_SYM: 8                                         (ferrum_dequant_int4_sym.rs:60)
 *   AWQ:      nibble(qzeros[g, n/8], awq_slot(n))       (awq_gemm_int4_typed.rs:203-205) */
int orc_zero_at(int fmt, const int32_t* qzeros, int N, int g, int n, int zero_offset);

/* Dequantised weight W16[k,n] as binary16 bits:
 *   RNE_f16( f32(q - z) * f32(scale[g,n]) ),  g = g_idx ? g_idx[k] : k / G
 * (w4a16_gptq_gemm_typed.rs:246-260; awq_gemm_int4_typed.rs:213-228).
 * out is row-major [K, N]. g_idx may be NULL. Returns 0, or -1 on bad g_idx. */
int orc_dequant(int fmt, const int32_t* qweight, const uint16_t* scales,
                const int32_t* qzeros, const int32_t* g_idx, int K, int N, int G,
                int zero_offset, uint16_t* out);

/* The standalone dequant kernels write the TRANSPOSED matrix out[n*K + k]
 * (ferrum_dequant_int4.rs:38-138, ferrum_dequant_int4_sym.rs:33-131). */
int orc_dequant_transposed(int fmt, const int32_t* qweight, const uint16_t* scales,
                           const int32_t* qzeros, const int32_t* g_idx, int K, int N,
                           int G, int zero_offset, uint16_t* out_nk);

/* out[m,n] = RNE_f16( sum_k f32(x[m,k]) * f32(w16[k,n]) ), the tt.dot f16 x f16 + f32
 * contraction (crates/triton-ir/src/dialect/tt.rs:143-150) followed by the store-time
 * truncf (w4a16_gptq_gemm_typed.rs:270-273). acc64 != 0 accumulates in double (the
 * exact-reference mode); otherwise in float in increasing k order.
 * out_f32 (optional) receives the unrounded sums. OpenMP over rows x columns. */
void orc_gemm_f16(const uint16_t* x, const uint16_t* w16, int M, int N, int K,
                  int acc64, uint16_t* out, float* out_f32);

/* Dequant + GEMM in one call (the reference CPU path: unpack -> dequant -> matmul). */
int orc_w4a16_gemm(int fmt, const uint16_t* x, const int32_t* qweight,
                   const uint16_t* scales, const int32_t* qzeros, const int32_t* g_idx,
                   int M, int N, int K, int G, int zero_offset, int acc64,
                   uint16_t* out, float* out_f32);

/* The bfloat16 instantiation (x, scales, W and out as bf16 bits): W = RNE_bf16(f32(q - z) *
 * f32(scale)), out = RNE_bf16(sum_k f32(x) * f32(W)); the reference kernels are generic over
 * the element type (w4a16_gptq_gemm_typed.rs:65-67). */
int orc_dequant_bf16(int fmt, const int32_t* qweight, const uint16_t* scales,
                     const int32_t* qzeros, const int32_t* g_idx, int K, int N, int G,
                     int zero_offset, uint16_t* out);
int orc_dequant_transposed_bf16(int fmt, const int32_t* qweight, const uint16_t* scales,
                                const int32_t* qzeros, const int32_t* g_idx, int K, int N,
                                int G, int zero_offset, uint16_t* out_nk);
int orc_w4a16_gemm_bf16(int fmt, const uint16_t* x, const int32_t* qweight,
                        const uint16_t* scales, const int32_t* qzeros, const int32_t* g_idx,
                        int M, int N, int K, int G, int zero_offset, int acc64,
                        uint16_t* out, float* out_f32);

/* Same, restricted to output rows `rows[0..nrows)` (a sample of a large M). */
int orc_w4a16_gemm_rows(int fmt, const uint16_t* x, const int32_t* qweight,
                        const uint16_t* scales, const int32_t* qzeros,
                        const int32_t* g_idx, int M, int N, int K, int G,
                        int zero_offset, const int32_t* rows, int nrows,
                        uint16_t* out /* [nrows, N] */);

/* ---- fused MoE (not in the reference; defined by composition) ---- */

/* softmax over E logits, top-k (ties -> lower expert index), weights renormalised to
 * sum to 1 over the selected k. ids/weights are [T, topk]. */
void orc_moe_route(const float* logits, int T, int E, int topk, int32_t* ids, float* weights);

/* Sort (token, slot) pairs by expert, stable in flattened pair index p = t*topk + j,
 * padding each expert's list to a multiple of block_m with the sentinel T*topk.
 * sorted_ids capacity must be >= T*topk + E*(block_m-1); expert_ids gets one entry
 * per block. Returns the padded length (num_tokens_post_padded). */
int orc_moe_align(const int32_t* ids, int T, int topk, int E, int block_m,
                  int32_t* sorted_ids, int32_t* expert_ids);

/* Full fused MoE layer, per token t:
 *   for each of its topk experts e with weight w:
 *     h1 = f16(x[t] @ W1_e), h3 = f16(x[t] @ W3_e)           (K -> I)
 *     a  = f16( silu(f32 h1) * f32 h3 )
 *     y_e = f16(a @ W2_e)                                      (I -> K)
 *   y[t] = f16( sum_j w_j * f32(y_e_j) )
 * Weights are per-expert w16 matrices (already dequantised), row-major:
 * w13[e] is [K, 2*I] with columns [0,I) = W1 and [I,2I) = W3; w2[e] is [I, K]. */
void orc_moe_forward(const uint16_t* x, int T, int K, int I, int E, int topk,
                     const int32_t* ids, const float* weights,
                     const uint16_t* const* w13, const uint16_t* const* w2, uint16_t* y);

/* silu(g) * u in f32 with the result rounded to f16 (crates/triton-kernels/src/
 * elementwise.rs:188-250 computes silu(x) = x / (1 + exp(-x)) in f32). */
uint16_t orc_silu_mul_f16(uint16_t g, uint16_t u);
/* The f32 twin (elementwise.rs:214-250), and the same over the interleaved layout: out[i]
 * for i < total, b = i / inter, from gate_up[b * 2 * inter + i % inter] and the element
 * inter further on. */
float orc_silu_mul_f32(float g, float u);
void orc_silu_mul_f32_rows(const float* gate_up, float* out, int inter, int64_t total);

/* Threads OpenMP will use (1 when built without OpenMP). */
int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
