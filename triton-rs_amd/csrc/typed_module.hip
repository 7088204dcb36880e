// Kernel-level drop-in code object (w4a16_typed.hsaco) for callers that drive the
// DeviceRuntime trait themselves: kernels named exactly like the reference's, with the
// reference's parameter list plus the two trailing scratch pointers Triton v3.6 appends
// (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:103-129,
//  awq_gemm_int4_typed.rs:94-115, crates/triton-runtime/examples/run_vec_add.rs:52-60).
// Launch: grid (cdiv(m, 64), cdiv(n, 64), 1), block (256, 1, 1), no dynamic LDS; the
// scratch pointers are accepted and ignored. w4a16_typed.json carries the same metadata
// fields as the reference's compile output (name, num_warps in 32-thread units,
// shared_mem, scratch sizes) plus the tile sizes.
#include "strided_body.h"

using namespace w4a16;

#define TYPED_PARAMS                                                                            \
    const half_t *a_ptr, const uint32_t *qweight_ptr, const half_t *scales_ptr,                \
        const uint32_t *qzeros_ptr, half_t *c_ptr, int m_size, int n_size, int k_size,         \
        int group_size, int stride_am, int stride_ak, int stride_qwk, int stride_qwn,          \
        int stride_sk, int stride_sn, int stride_qzk, int stride_qzn, int stride_cm,           \
        int stride_cn, void *global_scratch, void *profile_scratch

static __device__ __forceinline__ StridedParams make_params(TYPED_PARAMS, int zero_offset) {
    (void)global_scratch;
    (void)profile_scratch;
    StridedParams p;
    p.a = a_ptr; p.qweight = qweight_ptr; p.scales = scales_ptr; p.qzeros = qzeros_ptr;
    p.g_idx = nullptr; p.c = c_ptr;
    p.m = m_size; p.n = n_size; p.k = k_size; p.group_size = group_size;
    p.stride_am = stride_am; p.stride_ak = stride_ak; p.stride_qwk = stride_qwk;
    p.stride_qwn = stride_qwn; p.stride_sk = stride_sk; p.stride_sn = stride_sn;
    p.stride_qzk = stride_qzk; p.stride_qzn = stride_qzn; p.stride_cm = stride_cm;
    p.stride_cn = stride_cn; p.zero_offset = zero_offset;
    p.gate = nullptr; p.gate_want = 0;
    return p;
}

// Marks this code object as the library's own: hiprt_module_load looks it up, and hiprt_launch
// then runs the planned kernels for launches of the two kernels below that follow the launch
// contract above (same arguments, same results; see hiprt.cpp).
extern "C" __device__ const unsigned int w4a16_typed_module_marker = 0x57344131u;

extern "C" __global__ void __launch_bounds__(256) w4a16_gptq_gemm_typed(TYPED_PARAMS) {
    strided_gemm_body<FMT_GPTQ>(make_params(a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr,
                                            m_size, n_size, k_size, group_size, stride_am,
                                            stride_ak, stride_qwk, stride_qwn, stride_sk,
                                            stride_sn, stride_qzk, stride_qzn, stride_cm,
                                            stride_cn, global_scratch, profile_scratch, 1));
}

extern "C" __global__ void __launch_bounds__(256) awq_gemm_int4_typed(TYPED_PARAMS) {
    strided_gemm_body<FMT_AWQ>(make_params(a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr,
                                           m_size, n_size, k_size, group_size, stride_am,
                                           stride_ak, stride_qwk, stride_qwn, stride_sk,
                                           stride_sn, stride_qzk, stride_qzn, stride_cm,
                                           stride_cn, global_scratch, profile_scratch, 0));
}
