// Device-side helpers shared by the W4A16 kernels (gfx950, wave64).
//
// Numeric contract (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:246-260,
// awq_gemm_int4_typed.rs:213-228): a weight is W16 = RNE_f16(f32(q - z) * f32(s)).
// Because |q - z| <= 16 and s has an 11-bit significand, (q - z) * s is exact in f32, so
// one correctly rounded fp16 multiply of fp16(q - z) by s yields the same bits. The
// kernels build fp16(q) with the exponent trick: the bit pattern 0x6400 | q is the fp16
// number 1024 + q (ulp 1 in [1024, 2048)), and 0x6400 | (q << 4) is 1024 + 16 q.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int FMT_GPTQ = 0;
constexpr int FMT_GPTQ_SYM = 1;
constexpr int FMT_AWQ = 2;
// Nibble slot of row i (0..7) of a prepared word: (i >> 1) | ((i & 1) << 2), so that
// (w >> 4 j) & 0x000F000F holds rows (2 j, 2 j + 1).
__host__ __device__ constexpr int prep_slot(int i) { return (i >> 1) | ((i & 1) << 2); }

constexpr uint32_t MAGIC2 = 0x64006400u;  // (1024, 1024) as two fp16

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// v_perm_b32: result byte i = byte sel_i of the 8-byte value {hi:lo}; selectors 0..3 pick
// `lo`, 4..7 pick `hi`.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// A constant in a VGPR that the compiler cannot see through. (a & mask) | bits with both
// constants given this way is selected as one v_and_or_b32 (a VOP3 instruction on this
// target cannot encode two literals, so with literals the compiler emits v_and + v_or).
// Being an ordinary instruction, it is covered by the compiler's hazard handling: an
// inline-asm v_and_or_b32 is not, and its result read by an MFMA one instruction later is
// read stale. The asm has no side effects, so identical copies are merged and hoisted.
__device__ __forceinline__ uint32_t vconst(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
    return r;
}

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    return (a & mask) | bits;
}

// fp16 pair (1024 + nibble at bit 0, 1024 + nibble at bit 16) from v
__device__ __forceinline__ half2_t nib_pair(uint32_t v) {
    return as_h2(and_or(v, vconst(0x000F000Fu), vconst(MAGIC2)));
}
// same for the nibbles at bits 4 and 20, left in place: (1024 + 16 q_lo, 1024 + 16 q_hi)
__device__ __forceinline__ half2_t nib_pair16(uint32_t v) {
    return as_h2(and_or(v, vconst(0x00F000F0u), vconst(MAGIC2)));
}

// fp32 += a.x*b.x + a.y*b.y  (v_dot2c_f32_f16: f16 x f16 products, f32 accumulate)
__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}
// the same for bf16 pairs (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot2(bf16x2_t a, bf16x2_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
}

// bf16 pair (128 + nibble at bit 0, 128 + nibble at bit 16) from v: 0x4300 | q is the bf16
// number 128 + q (ulp 1 in [128, 256)). bf16 keeps 7 fraction bits, so a nibble must sit at
// bits 0..3 (no 16 q form as for fp16).
constexpr uint32_t MAGIC2_BF16 = 0x43004300u;   // (128, 128) as two bf16
__device__ __forceinline__ bf16x2_t nib_pair_bf16(uint32_t v) {
    return __builtin_bit_cast(bf16x2_t, and_or(v, vconst(0x000F000Fu), vconst(MAGIC2_BF16)));
}

// element pair type and the bias of the exponent trick per element type
template <typename E> struct pair2;
template <> struct pair2<half_t> { typedef half2_t type; static constexpr float bias = 1024.0f; };
template <> struct pair2<bf16_t> { typedef bf16x2_t type; static constexpr float bias = 128.0f; };

// 32 bits as an element pair. Take the word by value: __builtin_bit_cast applied directly to
// an element of an ext_vector_type value (v.y) reads element 0 with this compiler.
template <typename E>
__device__ __forceinline__ typename pair2<E>::type as_pair(uint32_t u) {
    return __builtin_bit_cast(typename pair2<E>::type, u);
}

// Nibble slot that column n occupies in an AWQ word: (n%8)/2 + (n%8)%2*4
// (awq_gemm_int4_typed.rs:139-151). Slot s is read from bits [4s, 4s+4).
__host__ __device__ constexpr int awq_slot(int n) { return ((n & 7) >> 1) + ((n & 1) << 2); }

// Column (within its 8-group) stored in AWQ slot s: the inverse of awq_slot.
__host__ __device__ constexpr int awq_col_of_slot(int s) { return ((s & 3) << 1) + (s >> 2); }

// Logical-shift nibble extract (arith.shrui + andi 0xF).
__device__ __forceinline__ int nib(uint32_t w, int slot) { return (int)((w >> (4 * slot)) & 0xFu); }

// Zero point for (group row `qz_row`, column n) under each format.
//   GPTQ: straight slot n%8, + zero_offset (+1 in the reference GEMM, :231-236)
//   GPTQ_SYM: 8 (ferrum_dequant_int4_sym.rs:60)
//   AWQ: slot awq_slot(n), no offset (awq_gemm_int4_typed.rs:203-205)
template <int FMT>
__device__ __forceinline__ int zero_of(uint32_t qz_word, int n, int zero_offset) {
    if constexpr (FMT == FMT_GPTQ_SYM) return 8;
    else if constexpr (FMT == FMT_AWQ) return nib(qz_word, awq_slot(n));
    else return nib(qz_word, n & 7) + zero_offset;
}

// Bit-exact dequant of one weight: RNE_f16((q - z) * s).
__device__ __forceinline__ half_t dequant1(int q, int z, half_t s) {
    return (half_t)(q - z) * s;
}

// The same for bfloat16 elements (the reference's kernels are generic over the element type,
// w4a16_gptq_gemm_typed.rs:65-67): RNE_bf16(f32(q - z) * f32(s)); a 5-bit integer times an
// 8-bit significand is exact in f32, so the only rounding is the final one to bf16.
__device__ __forceinline__ bf16_t dequant1(int q, int z, bf16_t s) {
    return (bf16_t)((float)(q - z) * (float)s);
}

// Two fp32 values as a packed element pair (low half first), each rounded to nearest even.
__device__ __forceinline__ uint32_t pack2(half_t, float a, float b) {
    return as_u32(half2_t{(half_t)a, (half_t)b});
}
__device__ __forceinline__ uint32_t pack2(bf16_t, float a, float b) {
    return __builtin_bit_cast(uint32_t, bf16x2_t{(bf16_t)a, (bf16_t)b});
}

// The bf16 pair RNE_bf16((q - z) * s) for the nibbles at bits 0 and 16 of v, given s and
// nzs = -z * s in fp32. q * s and z * s are exact in fp32 (a 5-bit integer times an 8-bit
// significand), so the fma returns (q - z) * s exactly and the pack rounds once: the same
// bits as dequant1 above. The byte conversions are v_cvt_f32_ubyte0 / ubyte2.
__device__ __forceinline__ uint32_t deq2_bf16(uint32_t v, float s, float nzs) {
    const uint32_t x = v & 0x000F000Fu;
    return pack2(bf16_t{}, __builtin_fmaf((float)(x & 0xFFu), s, nzs),
                 __builtin_fmaf((float)(x >> 16), s, nzs));
}

// bf16 bits (low 16 bits of b) as fp32: exact
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// v_mfma_f32_16x16x32 for either element type
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8-element vector of an element type
template <typename E> struct vec8;
template <> struct vec8<half_t> { typedef half8_t type; };
template <> struct vec8<bf16_t> { typedef bf16x8_t type; };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// base + byte offset with a 32-bit offset: lets the compiler use the global_load
// "v_offset, s_base" form instead of a 64-bit address add per load
template <typename T>
__device__ __forceinline__ const T* at_bytes(const T* base, uint32_t byte_off) {
    return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Buffer resource over [base, base + bytes) (raw buffer, no swizzle; gfx9 word 3) and loads
// through it: address = base + voffset (per lane) + soffset (uniform, an SGPR), so a wave
// streaming rows of a matrix keeps one per-lane offset and adds the row offset on the scalar
// unit. aux = 2 is the non-temporal (streaming) hint. Out-of-range offsets read zero.
typedef __amdgpu_buffer_rsrc_t bufrsrc_t;
__device__ __forceinline__ bufrsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t buf_ld_stream(bufrsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 2);
}

// Streaming (non-temporal) loads for packed weights, which are read exactly once.
__device__ __forceinline__ uint32_t ld_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ u32x2 ld_stream2(const uint32_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ u32x4 ld_stream4(const uint32_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// silu(g) * u with g, u and the result in f32 (crates/triton-kernels/src/elementwise.rs:
// 214-250): denominator exp(-g) + 1, one division, one product, each rounded to f32 (no
// contraction).
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
#pragma clang fp contract(off)
    const float s = g / (expf(-g) + 1.0f);
    return s * u;
}

// f16(silu(g) * u) with g, u fp16 and silu(g) = g / (1 + exp(-g)) in f32
// (crates/triton-kernels/src/elementwise.rs:188-212): the product is rounded to f32, then to
// f16, as in the reference and the oracle. Contraction is off and the product passes through
// an empty asm: otherwise the compiler may fold multiply and conversion into one
// mixed-precision FMA (v_fma_mixlo_f16), which rounds once and differs from the two
// roundings in about 1 case in 15000 (seen where the code was inlined into a GEMM epilogue).
__device__ __forceinline__ half_t silu_mul_f16(half_t g, half_t u) {
#pragma clang fp contract(off)
    const float gf = (float)g;
    const float s = gf / (1.0f + expf(-gf));
    float prod = s * (float)u;
    asm volatile("" : "+v"(prod));
    return (half_t)prod;
}

}  // namespace w4a16
