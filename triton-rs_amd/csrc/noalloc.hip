// Allocation-free variant of w4a16_gemm (w4a16_gemm_noalloc) for callers that cannot call
// hipMalloc: code under HIP graph capture, tight serving loops, harnesses that forbid
// allocation. The split-K scratch of its kernels (tile counters, the fixed-point hand-off's
// slot words and split masks, fp32 partials) lives in one file-scope device array of fixed
// size instead of the per-stream workspace w4a16_gemm grows on demand.
//
// The array's name is a host-side stand-in in host code: its device address is taken once
// per device with hipGetSymbolAddress (w4a16_init, or the entry point's first call on the
// device) and only that address is handed to kernels. Each device holds its own copy for the
// life of the process. Every call on a device shares that device's copy: calls that overlap
// in time on one device (two streams, or two threads) race and must be serialised by the
// caller. The kernels leave counters, slots and masks at zero after every call; set-up clears
// them once with a fill kernel.
#include <map>
#include <mutex>

#include "../../include/w4a16.h"
#include "launch.h"

namespace w4a16 {

// Layout of the scratch array (bytes):
//   [0, NA_COUNTER_BYTES)              tile counters, FLAG_STRIDE words apart (NA_MAX_TILES)
//   then FIX_MAX_ENTRIES 64-bit slot words, then FIX_MAX_ENTRIES 32-bit split masks
//   then NA_PARTIAL_BYTES of fp32 partials
constexpr size_t NA_MAX_TILES = 1024;
constexpr size_t NA_COUNTER_BYTES = NA_MAX_TILES * FLAG_STRIDE * sizeof(uint32_t);   // 256 KiB
constexpr size_t NA_ZERO_BYTES = NA_COUNTER_BYTES + FIX_SLOT_BYTES;                  // 1.09 MiB
constexpr size_t NA_SCRATCH_BYTES = 8u << 20;
constexpr size_t NA_PARTIAL_BYTES = NA_SCRATCH_BYTES - NA_ZERO_BYTES;               // 6.9 MiB
static_assert(NA_ZERO_BYTES % 256 == 0, "partials stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[NA_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) zero_words(uint4* p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

static std::mutex g_na_mu;
static std::map<int, unsigned char*> g_na_ptr;   // device -> address of that device's `scratch`

// Once per device, with the device current: look the array up and clear what must start at
// zero. The clear is enqueued on `st` (the caller's stream, ahead of its kernels); from
// w4a16_init (st = null stream) it is waited for.
int noalloc_setup(hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (g_na_ptr.count(dev)) return W4A16_OK;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, static_cast<uint4*>(ptr),
                       NA_ZERO_BYTES / 16);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "scratch clear launch");
    if (!st && (e = hipStreamSynchronize(nullptr)) != hipSuccess)
        return hip_fail(e, "hipStreamSynchronize");
    g_na_ptr[dev] = static_cast<unsigned char*>(ptr);
    return W4A16_OK;
}

static int noalloc_scratch(hipStream_t st, size_t partial_bytes, Scratch* out) {
    (void)partial_bytes;   // checked against NA_PARTIAL_BYTES by the caller
    if (int rc = noalloc_setup(st)) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    unsigned char* base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_na_mu);
        base = g_na_ptr[dev];
    }
    out->counters = reinterpret_cast<uint32_t*>(base);
    out->slots = reinterpret_cast<uint64_t*>(base + NA_COUNTER_BYTES);
    out->masks = reinterpret_cast<uint32_t*>(out->slots + FIX_MAX_ENTRIES);
    out->partials = reinterpret_cast<float*>(base + NA_ZERO_BYTES);
    return W4A16_OK;
}

static const ScratchSource NOALLOC_SCRATCH = {NA_PARTIAL_BYTES, NA_MAX_TILES, false, false, noalloc_scratch};

}  // namespace w4a16

extern "C" {

W4A16_API size_t w4a16_gemm_noalloc_scratch_bytes(void) { return w4a16::NA_SCRATCH_BYTES; }

W4A16_API int w4a16_gemm_noalloc(void* stream, int fmt, const void* x, const void* qweight,
                                 const void* scales, const void* qzeros, const int32_t* g_idx,
                                 void* out, int32_t M, int32_t N, int32_t K, int32_t group_size,
                                 int32_t gptq_zero_offset) {
    return w4a16::gemm_impl(stream, fmt, x, qweight, scales, qzeros, g_idx, out, M, N, K,
                            group_size, gptq_zero_offset, w4a16::NOALLOC_SCRATCH);
}

}  // extern "C"
