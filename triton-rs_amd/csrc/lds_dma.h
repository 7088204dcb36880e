// Buffer loads that write straight into LDS (buffer_load_dwordx4 ... lds) and the helpers
// around them, shared by the kernels that stage operands this way.
#pragma once
#include "device_common.h"

namespace w4a16 {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over [base, base + bytes) in scalar registers (gfx9 word 3: no
// swizzle, 32-bit data format). Offsets at or past `bytes` read zero.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return i32x4_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                   __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu)),
                   __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// LDS byte address of a pointer into the kernel's dynamic LDS
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>(
        (__attribute__((address_space(3))) const char*)(p));
}

// buffer_load_dwordx4 ... lds: 16 bytes per lane from rsrc + voffset into LDS at M0 (the
// wave's base) + lane * 16. Issued from asm so that the compiler, which cannot tell the ring
// slots apart, does not wait for every LDS load before each LDS read; the kernel counts these
// loads itself (vmcnt). s_nop: one wait state between the M0 write and its use. "memory":
// the compiler must not move LDS accesses across it or assume the LDS unchanged.
__device__ __forceinline__ void dma16(i32x4_t rsrc, const void* lds_wave_base, uint32_t voffset) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
    uint32_t saved;
    // M0 is reserved to the compiler: saved and restored around the load
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(voffset), "s"(rsrc)
        : "memory");
}

// s_waitcnt vmcnt(n) leaving lgkmcnt and expcnt alone (gfx9 encoding: vmcnt in [3:0] and
// [15:14])
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

constexpr uint32_t DMA_OOB = 0x80000000u;   // voffset of a zero (past any buffer)

}  // namespace w4a16
