// C-ABI op layer: argument validation (before any HIP call), kernel selection, split-K
// workspace management and error reporting for include/w4a16.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/w4a16.h"
#include "launch.h"

namespace w4a16 {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(W4A16_ERR_DEVICE, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

static inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ------------------------------------------------------------------ workspace

// One split-K workspace per (device, stream): per-tile counters (zeroed at allocation,
// returned to zero by the kernels themselves) followed by fp32 partials. A workspace is
// never freed: HIP graphs captured on the stream keep its address in their kernel nodes,
// so when a larger request arrives a new buffer takes its place and the old one is retired
// (kept allocated until the process ends). Growth allocates memory, which graph capture
// forbids; under capture a call that would need a larger workspace fails with an error
// asking for one call of that size outside capture first.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
};
static std::mutex g_ws_mu;
static std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
static std::vector<void*> g_ws_retired;   // superseded workspaces, alive until exit

// room for SPLITK_MAX_TILES counters, then the fixed-point hand-off's slots and masks
constexpr size_t COUNTER_BYTES = SPLITK_FLAG_BYTES + FIX_SLOT_BYTES;

static bool stream_capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) { (void)hipGetLastError(); return false; }
    return cs != hipStreamCaptureStatusNone;
}

// The buffer of `map` for the current device and stream, at least `need` bytes; a new one
// (first `zero` bytes cleared, ordered on the stream) replaces a smaller one, which is retired.
static int stream_buffer(std::map<std::pair<int, hipStream_t>, Workspace>& map, hipStream_t st,
                         size_t need, size_t zero, const char* what, void** base) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = map[{dev, st}];
    if (w.bytes < need) {
        if (stream_capturing(st))
            return fail(W4A16_ERR_UNSUPPORTED,
                        "%s of %zu bytes needed while the stream is being captured: "
                        "make one call of this size on the stream before capturing", what, need);
        const size_t grow = need < (size_t)(8 << 20) ? (size_t)(8 << 20) : need;
        void* fresh = nullptr;
        e = hipMalloc(&fresh, grow);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
        if (zero) {
            // ordered after everything queued on the stream, before this call's kernels
            e = hipMemsetAsync(fresh, 0, zero, st);
            if (e != hipSuccess) { (void)hipFree(fresh); return hip_fail(e, "hipMemsetAsync(workspace)"); }
        }
        if (w.base) g_ws_retired.push_back(w.base);
        w.base = fresh;
        w.bytes = grow;
    }
    *base = w.base;
    return W4A16_OK;
}

static int get_workspace(hipStream_t st, size_t need, uint32_t** counters, float** partials) {
    void* base = nullptr;
    if (int rc = stream_buffer(g_ws, st, COUNTER_BYTES + need, COUNTER_BYTES, "split-K workspace", &base))
        return rc;
    *counters = static_cast<uint32_t*>(base);
    *partials = reinterpret_cast<float*>(static_cast<char*>(base) + COUNTER_BYTES);
    return W4A16_OK;
}

// Per-(device, stream) buffer for activations gathered into act-order group order.
static std::map<std::pair<int, hipStream_t>, Workspace> g_gather;
// act-order beyond 64 rows on w4a16_gemm: perm, the gate word and the repacked rows
static std::map<std::pair<int, hipStream_t>, Workspace> g_actorder;

// ------------------------------------------------------------------ validation

static int check_gemm_args(int fmt, const void* x, const void* qweight, const void* scales,
                           const void* qzeros, const void* out, int32_t M, int32_t N,
                           int32_t K, int32_t G) {
    if (fmt != W4A16_FMT_GPTQ && fmt != W4A16_FMT_GPTQ_SYM && fmt != W4A16_FMT_AWQ)
        return fail(W4A16_ERR_INVALID_ARG, "unknown weight format %d", fmt);
    if (!x || !qweight || !scales || !out)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument (x, qweight, scales or out)");
    if (fmt != W4A16_FMT_GPTQ_SYM && !qzeros)
        return fail(W4A16_ERR_INVALID_ARG, "qzeros is required for GPTQ and AWQ formats");
    if (M < 1 || N < 1 || K < 1 || G < 1)
        return fail(W4A16_ERR_INVALID_ARG, "sizes must be positive (M=%d N=%d K=%d group_size=%d)",
                    M, N, K, G);
    if (K % G)
        return fail(W4A16_ERR_INVALID_ARG, "K (%d) must be a multiple of group_size (%d)", K, G);
    if (N % 8)
        return fail(W4A16_ERR_INVALID_ARG, "N (%d) must be a multiple of 8 (packed qzeros / AWQ)", N);
    if (fmt != W4A16_FMT_AWQ && K % 8)
        return fail(W4A16_ERR_INVALID_ARG, "K (%d) must be a multiple of 8 for GPTQ packing", K);
    return W4A16_OK;
}

// GPTQ zero point = nibble + zero_offset: 1 for the reference's GEMM, 0 for its dequant
// kernel. The kernels form fp16(1024 + zero) exactly for zeros up to 1023; the accepted
// range is kept to what a packed format can mean.
static int check_zero_offset(int fmt, int32_t zero_offset) {
    if (fmt == W4A16_FMT_GPTQ && (zero_offset < 0 || zero_offset > 16))
        return fail(W4A16_ERR_INVALID_ARG, "gptq_zero_offset %d outside [0, 16]", zero_offset);
    return W4A16_OK;
}

constexpr int DEFAULT_CUS = 256;  // MI355X

// Compute units of the current device (cached per device; 256 when it cannot be queried).
static int device_cus() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { (void)hipGetLastError(); return DEFAULT_CUS; }
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
        (void)hipGetLastError();
        cus = DEFAULT_CUS;
    }
    cache[dev] = cus;
    return cus;
}

// Whether workgroup b of a launch runs on XCD b mod 8 on the current device (the GEMV's
// L2-local split-K hand-off relies on it). Probed once per device with a small synchronous
// kernel; false when the probe fails or placement differs, and the kernels then use the
// device-scope hand-off. The probe allocates and synchronises, which graph capture forbids:
// a call made while its stream is being captured, before the device was probed, takes the
// device-scope variant (correct everywhere) and leaves the probe for a later call.
// w4a16_init() runs the probe up front.
static bool xcd_placement(hipStream_t st, bool probe = true) {
    static std::mutex mu;
    static std::map<int, bool> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { (void)hipGetLastError(); return false; }
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    if (!probe || stream_capturing(st)) return false;
    bool ok = false;
    if (check_xcd_placement(&ok) != hipSuccess) { (void)hipGetLastError(); ok = false; }
    cache[dev] = ok;
    return ok;
}

// The placement result if this device has been probed, else false (no probe).
static bool xcd_placement_cached() {
    return xcd_placement(nullptr, /*probe=*/false);
}

// Act-order beyond the small-batch kernel: the per-call group order (act_order.hip) feeds the
// prefill kernel; it needs K <= 32768 and at most 1024 groups.
static bool act_order_prefill_ok(int fmt, int M, int N, int K, int G, int cus, bool bf16 = false) {
    if (!(fmt == W4A16_FMT_GPTQ || fmt == W4A16_FMT_GPTQ_SYM) || K > 32768 || K % G || K / G > 1024)
        return false;
    const PrefillShape ps = prefill_shape(fmt, M, N, K, G, cus);
    return ps.ok && (!bf16 || ps.dma);   // bf16 runs the pipelined prefill only
}

// Act-order from 65 to 128 rows: the direct-x small-batch kernel on the checkpoint as stored
// (per-workgroup (scale, zero) table, no scratch) over two row chunks, 64 and M - 64. Each
// chunk reads all the weights, which at these sizes costs less than the group-order route's
// per-call staging (order, repack and gather, ~15 us at K = 4096, N = 6144, where M = 96 /
// 128 took 42.3 / 44.8 us through the route).
static bool act_order_chunks_ok(int fmt, int M, int N, int K, int G) {
    return M > 64 && M <= 128 && ck_frag_shape(fmt, 64, N, K, G, true).ok &&
           ck_frag_shape(fmt, M - 64, N, K, G, true).ok;
}

static int plan(int fmt, int M, int N, int K, int G, bool has_gidx, int cus = DEFAULT_CUS) {
    if (has_gidx) {
        const SkinnyShape sk = skinny_shape(fmt, M, N, K, G, cus, true);
        if (sk.ok && (size_t)sk.col_tiles <= SPLITK_MAX_TILES) return W4A16_KERNEL_SKINNY;
        if (act_order_chunks_ok(fmt, M, N, K, G)) return W4A16_KERNEL_SKINNY;
        return act_order_prefill_ok(fmt, M, N, K, G, cus) ? W4A16_KERNEL_PREFILL : W4A16_KERNEL_STRIDED;
    }
    const GemvShape gv = gemv_shape(fmt, M, N, K, G, false);
    if (gv.ok && (size_t)gv.col_tiles <= SPLITK_MAX_TILES) return W4A16_KERNEL_GEMV;
    const SkinnyShape sk = skinny_shape(fmt, M, N, K, G, cus);
    if (M <= 64 && sk.ok && (size_t)sk.col_tiles <= SPLITK_MAX_TILES)
        return W4A16_KERNEL_SKINNY;
    if (prefill_shape(fmt, M, N, K, G, cus).ok) return W4A16_KERNEL_PREFILL;
    return W4A16_KERNEL_STRIDED;
}

// bfloat16 elements (W4A16_BF16): the VALU GEMVs (and the row-paired AWQ one up to 8 rows),
// the small-batch kernel up to 64 and the pipelined prefill beyond, on the checkpoint
// layouts; act-order as for fp16 (small-batch table, else the group-order prefill route); the
// shapes those kernels reject run the generic kernel.
static int plan_bf16(int fmt, int M, int N, int K, int G, bool has_gidx, int cus = DEFAULT_CUS) {
    if (has_gidx) {
        const SkinnyShape sk = skinny_shape(fmt, M, N, K, G, cus, true);
        if (sk.ok && (size_t)sk.col_tiles <= SPLITK_MAX_TILES) return W4A16_KERNEL_SKINNY;
        return act_order_prefill_ok(fmt, M, N, K, G, cus, true) ? W4A16_KERNEL_PREFILL : W4A16_KERNEL_STRIDED;
    }
    const GemvShape gv = gemv_shape(fmt, M, N, K, G, false, /*bf16=*/true);
    if (gv.ok && (size_t)gv.col_tiles <= SPLITK_MAX_TILES) return W4A16_KERNEL_GEMV;
    const SkinnyShape sk = skinny_shape(fmt, M, N, K, G, cus);
    if (M <= 64 && sk.ok && (size_t)sk.col_tiles <= SPLITK_MAX_TILES) return W4A16_KERNEL_SKINNY;
    const PrefillShape ps = prefill_shape(fmt, M, N, K, G, cus);
    return ps.ok && ps.dma ? W4A16_KERNEL_PREFILL : W4A16_KERNEL_STRIDED;
}

}  // namespace w4a16

using namespace w4a16;

extern "C" {

W4A16_API const char* w4a16_last_error(void) { return g_last_error.c_str(); }

W4A16_API const char* w4a16_version(void) { return "w4a16-mi355x 0.2 (gfx950)"; }

W4A16_API int w4a16_init(int32_t device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) {
        (void)hipGetLastError();
        return fail(W4A16_ERR_BACKEND_DISABLED, "no HIP device available");
    }
    if (device < 0 || device >= n)
        return fail(W4A16_ERR_INVALID_ARG, "device %d outside [0, %d)", device, n);
    int prev = 0;
    e = hipGetDevice(&prev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (prev != device && (e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    (void)device_cus();
    (void)xcd_placement(nullptr);
    if (int rc = noalloc_setup(nullptr)) {
        if (prev != device) (void)hipSetDevice(prev);
        return rc;
    }
    if (prev != device && (e = hipSetDevice(prev)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    return W4A16_OK;
}

W4A16_API int w4a16_gemm_plan(int fmt, int32_t M, int32_t N, int32_t K, int32_t G, int has_g_idx,
                              int* kernel) {
    const bool bf16 = (fmt & W4A16_BF16) != 0;
    fmt &= ~W4A16_BF16;
    int rc = check_gemm_args(fmt, (void*)1, (void*)1, (void*)1, (void*)1, (void*)1, M, N, K, G);
    if (rc) return rc;
    if (!kernel) return fail(W4A16_ERR_INVALID_ARG, "kernel out-pointer is null");
    *kernel = bf16 ? plan_bf16(fmt, M, N, K, G, has_g_idx != 0) : plan(fmt, M, N, K, G, has_g_idx != 0);
    return W4A16_OK;
}

}  // extern "C"

namespace w4a16 {

// Scratch of the per-stream allocated workspace (get_workspace), sized on demand.
static int alloc_scratch(hipStream_t st, size_t partial_bytes, Scratch* out) {
    uint32_t* counters = nullptr;
    float* partials = nullptr;
    if (int rc = get_workspace(st, partial_bytes, &counters, &partials)) return rc;
    out->counters = counters;
    out->slots = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(counters) + SPLITK_FLAG_BYTES);
    out->masks = reinterpret_cast<uint32_t*>(out->slots + FIX_MAX_ENTRIES);
    out->partials = partials;
    return W4A16_OK;
}

ScratchSource alloc_scratch_source() { return ScratchSource{SIZE_MAX, SPLITK_MAX_TILES, true, true, alloc_scratch}; }

int gemm_impl(void* stream, int fmt, const void* x, const void* qweight, const void* scales,
              const void* qzeros, const int32_t* g_idx, void* out, int32_t M, int32_t N,
              int32_t K, int32_t G, int32_t zero_offset, const ScratchSource& src) {
    const bool bf16 = (fmt & W4A16_BF16) != 0;
    fmt &= ~W4A16_BF16;
    int rc = check_gemm_args(fmt, x, qweight, scales, qzeros, out, M, N, K, G);
    if (!rc) rc = check_zero_offset(fmt, zero_offset);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool vec_ok = aligned(x, 16) && aligned(qweight, 16) && aligned(scales, 16) &&
                        aligned(out, 16) && (!qzeros || aligned(qzeros, 16)) &&
                        (!g_idx || aligned(g_idx, 16));
    const int cus = device_cus();
    int kernel = bf16 ? plan_bf16(fmt, M, N, K, G, g_idx != nullptr, cus)
                      : plan(fmt, M, N, K, G, g_idx != nullptr, cus);
    if (!vec_ok) kernel = W4A16_KERNEL_STRIDED;
    if (g_idx && kernel == W4A16_KERNEL_PREFILL && !src.may_allocate) kernel = W4A16_KERNEL_STRIDED;
    // GPTQ small batches beyond 16 rows (plain order also 9..16 with 64-column workgroups;
    // act-order also any M >= 2 with groups under 128 rows): the direct-x small-batch kernel on
    // the checkpoint as stored (one workgroup over all of K for its columns: no split-K
    // hand-off, no scratch; act-order through a per-workgroup (scale, zero) table). Act-order,
    // same-box A/B against the split-K kernel's table path, K=4096 -> N=6144: M = 32 / 48 / 64
    // 12.30 / 16.34 / 17.03 -> 11.35 / 13.26 / 14.79 us; G = 32 M = 16 / 64 16.81 / 17.45 ->
    // 11.40 / 15.26 us; up to 16 rows at G = 128 slower (M = 2 / 8 / 16 7.95 / 9.15 / 9.77 ->
    // 10.40 / 10.50 / 10.84 us: its per-row table reads, ~4 bytes of LDS per weight, fall on
    // 192 workgroups). Plain order, same-box A/B against the split-K kernel,
    // K=4096 -> N=6144: M = 32 / 48 / 64 11.12 / 14.62 / 15.38 -> 10.18 / 13.12 / 14.67 us;
    // M = 16 on N = 14336 (4 columns per lane) 13.42 -> 12.42 us; 14336 -> 4096 M = 32
    // 26.17 -> 25.86 us. Up to 16 rows with 32-column workgroups it was slower (M = 9 / 16
    // 7.55 / 8.35 -> 8.25 / 8.45 us, 8192 x 8192 M = 16 13.49 -> 14.35 us): its workgroups
    // read 128-byte pieces of K / 8 packed rows N * 4 bytes apart, where the prepared layout
    // streams whole strips (6.05 us at config 2's M = 16); 16- and 64-column workgroups were
    // slower still.
    if (kernel == W4A16_KERNEL_SKINNY && g_idx && !bf16 && M > 64) {   // act_order_chunks_ok
        for (int m0 = 0; m0 < M; m0 += 64) {
            const int rows = M - m0 < 64 ? M - m0 : 64;
            const PrepFragShape fs = ck_frag_shape(fmt, rows, N, K, G, true);
            PrepFragParams p{};
            p.g_idx = g_idx;
            p.x = static_cast<const half_t*>(x) + (size_t)m0 * K;
            p.qweight = static_cast<const uint32_t*>(qweight);
            p.scales = static_cast<const half_t*>(scales);
            p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
            p.zero_offset = zero_offset;
            p.out = static_cast<half_t*>(out) + (size_t)m0 * N;
            p.M = rows; p.N = N; p.K = K; p.G = G;
            hipError_t e = launch_ck_frag(fmt, p, fs, st);
            if (e != hipSuccess) return hip_fail(e, "small-batch launch");
        }
        return W4A16_OK;
    }
    if (kernel == W4A16_KERNEL_SKINNY && !bf16 && fmt != W4A16_FMT_AWQ && (g_idx ? M >= 2 : M > 8)) {
        const PrepFragShape fs = ck_frag_shape(fmt, M, N, K, G, g_idx != nullptr);
        if (fs.ok && (g_idx ? M > 16 || G < 128 : M > 16 || fs.s == 4)) {
            PrepFragParams p{};
            p.g_idx = g_idx;
            p.x = static_cast<const half_t*>(x);
            p.qweight = static_cast<const uint32_t*>(qweight);
            p.scales = static_cast<const half_t*>(scales);
            p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
            p.zero_offset = zero_offset;
            p.out = static_cast<half_t*>(out);
            p.M = M; p.N = N; p.K = K; p.G = G;
            hipError_t e = launch_ck_frag(fmt, p, fs, st);
            return e == hipSuccess ? W4A16_OK : hip_fail(e, "small-batch launch");
        }
    }
    // the placement probe allocates: sources that must not allocate use what is cached
    const bool xcd = src.may_probe ? xcd_placement(st) : xcd_placement_cached();
    auto scratch_for = [&](size_t tiles, size_t partial_bytes, Scratch* sc) -> int {
        if (tiles > src.max_tiles)
            return fail(W4A16_ERR_UNSUPPORTED, "%zu split-K tiles exceed the counter area (%zu)",
                        tiles, src.max_tiles);
        if (partial_bytes > src.max_partial_bytes)
            return fail(W4A16_ERR_UNSUPPORTED,
                        "split-K partials of %zu bytes exceed the scratch limit of %zu bytes "
                        "(M=%d N=%d K=%d)", partial_bytes, src.max_partial_bytes, M, N, K);
        return src.get(st, partial_bytes, sc);
    };
    // A fixed scratch area (w4a16_gemm_noalloc) may be too small for the split-K partials of
    // the planned GEMV or small-batch kernel (e.g. AWQ M = 8 on a 70B-class MLP: 7 MiB): such
    // a call takes the prefill kernel instead, with the largest K split whose partials fit
    // (run_prefill), down to none, which needs no scratch.
    auto scratch_fits = [&](size_t tiles, size_t partial_bytes) {
        return tiles <= src.max_tiles && partial_bytes <= src.max_partial_bytes;
    };
    auto unsplit_prefill_ok = [&]() {   // bf16 runs the pipelined prefill only
        const PrefillShape q = prefill_shape(fmt, M, N, K, G, cus, 1);
        return q.ok && (!bf16 || q.dma);
    };
    if (kernel == W4A16_KERNEL_SKINNY) {
        const SkinnyShape s = skinny_shape(fmt, M, N, K, G, cus, g_idx != nullptr, xcd);
        if (s.splits > 1 && !scratch_fits((size_t)s.col_tiles, (size_t)s.splits * M * N * sizeof(float)))
            kernel = g_idx ? W4A16_KERNEL_STRIDED
                           : unsplit_prefill_ok() ? W4A16_KERNEL_PREFILL : W4A16_KERNEL_STRIDED;
    } else if (kernel == W4A16_KERNEL_GEMV) {
        const GemvShape s = gemv_shape(fmt, M, N, K, G, xcd, bf16);
        if (s.splits > 1 && !scratch_fits((size_t)s.col_tiles, (size_t)s.splits * M * N * sizeof(float)))
            kernel = unsplit_prefill_ok() ? W4A16_KERNEL_PREFILL : W4A16_KERNEL_STRIDED;
    }

    if (kernel == W4A16_KERNEL_SKINNY) {
        const SkinnyShape s = skinny_shape(fmt, M, N, K, G, cus, g_idx != nullptr, xcd);
        SkinnyParams p{};
        p.g_idx = g_idx;
        p.x = static_cast<const half_t*>(x);
        p.qweight = static_cast<const uint32_t*>(qweight);
        p.scales = static_cast<const half_t*>(scales);
        p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G; p.zero_offset = zero_offset;
        p.splits = s.splits; p.steps_per_wave = s.steps_per_wave; p.col_tiles = s.col_tiles;
        if (s.splits > 1) {
            Scratch sc{};
            rc = scratch_for((size_t)s.col_tiles, (size_t)s.splits * M * N * sizeof(float), &sc);
            if (rc) return rc;
            p.flags = sc.counters;
            p.ws = sc.partials;
        }
        hipError_t e = launch_skinny(fmt, p, s, st, bf16);
        if (e != hipSuccess) return hip_fail(e, "skinny launch");
        return W4A16_OK;
    }

    // the prefill kernel on (xp, qwp) with the call's scales and zeros; gate as PrefillParams
    auto run_prefill = [&](const void* xp, const void* qwp, const uint32_t* gate) -> int {
        // a fixed scratch area too small for the planned split's partials: the best plan with
        // at most half the splits, down to none (no scratch at all)
        PrefillShape s = prefill_shape(fmt, M, N, K, G, cus);
        while (s.ksplit > 1 && ((size_t)s.ksplit * M * N * sizeof(float) > src.max_partial_bytes ||
                                (size_t)s.col_tiles * s.row_tiles > src.max_tiles))
            s = prefill_shape(fmt, M, N, K, G, cus, s.ksplit / 2);
        PrefillParams p{};
        p.x = static_cast<const half_t*>(xp);
        p.qweight = static_cast<const uint32_t*>(qwp);
        p.scales = static_cast<const half_t*>(scales);
        p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G; p.zero_offset = zero_offset;
        p.ksplit = s.ksplit;
        p.gate = gate;
        p.gate_want = 1;
        if (s.ksplit > 1) {
            Scratch sc{};
            const int r = scratch_for((size_t)s.col_tiles * s.row_tiles,
                                      (size_t)s.ksplit * M * N * sizeof(float), &sc);
            if (r) return r;
            p.counters = sc.counters;
            p.ws = sc.partials;
        }
        hipError_t e = launch_prefill(fmt, p, s, st, bf16);
        return e == hipSuccess ? W4A16_OK : hip_fail(e, "prefill launch");
    };
    if (kernel == W4A16_KERNEL_PREFILL && !g_idx) return run_prefill(x, qweight, nullptr);

    // act-order beyond the small-batch kernel's rows: per call, the group order of the rows is
    // computed on the device (perm, and a gate word that is 1 when every group holds exactly G
    // rows; kept from the stream's previous call when g_idx, K and G are the same), the packed
    // rows are repacked into it and x's columns gathered by it (one launch), then the
    // prefill kernel runs on them when the gate is 1 and the generic kernel on the checkpoint
    // when it is 0 (each reads the gate and returns at once when it is not the one wanted).
    // Without the per-stream buffers (allocation-free entry) the generic kernel alone runs.
    const uint32_t* gate = nullptr;
    if (kernel == W4A16_KERNEL_PREFILL) {
        const size_t perm_bytes = ((size_t)K * 4 + 255) & ~(size_t)255;
        void* ws = nullptr;
        void* xg = nullptr;
        // [header 256 B: gate word, then the order's memo (valid, K, G); cleared when the
        //  buffer is allocated][perm][copy of the g_idx perm was computed from][repacked rows]
        rc = stream_buffer(g_actorder, st, 256 + 2 * perm_bytes + (size_t)K / 8 * N * 4, 256, "act-order repack buffer", &ws);
        if (!rc) rc = stream_buffer(g_gather, st, (size_t)M * K * sizeof(half_t), 0, "act-order gather buffer", &xg);
        if (rc) return rc;
        uint32_t* gw = static_cast<uint32_t*>(ws);
        int32_t* perm = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + 256);
        int32_t* gcopy = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + 256 + perm_bytes);
        uint32_t* qout = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + 256 + 2 * perm_bytes);
        hipError_t e = launch_act_order_perm(g_idx, perm, gw, gcopy, K, G, st);
        if (e == hipSuccess)
            e = launch_act_order_stage(static_cast<const uint32_t*>(qweight), perm, qout,
                                       static_cast<const half_t*>(x), static_cast<half_t*>(xg), M, K, N, st);
        if (e != hipSuccess) return hip_fail(e, "act-order group order launch");
        if ((rc = run_prefill(xg, qout, gw))) return rc;
        gate = gw;
    }

    if (kernel == W4A16_KERNEL_GEMV) {
        const GemvShape s = gemv_shape(fmt, M, N, K, G, xcd, bf16);
        GemvParams p{};
        p.x = static_cast<const half_t*>(x);
        p.qweight = static_cast<const uint32_t*>(qweight);
        p.scales = static_cast<const half_t*>(scales);
        p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G; p.zero_offset = zero_offset; p.splits = s.splits;
        p.col_tiles = s.col_tiles;
        if (s.splits > 1) {
            Scratch sc{};
            rc = scratch_for((size_t)s.col_tiles, (size_t)s.splits * M * N * sizeof(float), &sc);
            if (rc) return rc;
            p.counters = sc.counters;
            p.ws = sc.partials;
            // every GEMV kernel takes the fixed-point hand-off where its limits allow
            const size_t entries = (size_t)M * N;
            p.fixed = s.splits <= FIX_MAX_SPLITS &&
                      ((M <= FIX_MAX_M && entries <= FIX_VALU_MAX_ENTRIES) ||
                       (s.awq_rows && entries <= FIX_MAX_ENTRIES));
            p.slots = sc.slots;
            p.masks = sc.masks;
        }
        hipError_t e = launch_gemv(fmt, p, s, st, bf16);
        if (e != hipSuccess) return hip_fail(e, "gemv launch");
        return W4A16_OK;
    }

    StridedParams p{};
    p.a = static_cast<const half_t*>(x);
    p.qweight = static_cast<const uint32_t*>(qweight);
    p.scales = static_cast<const half_t*>(scales);
    p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
    p.g_idx = g_idx;
    p.c = static_cast<half_t*>(out);
    p.m = M; p.n = N; p.k = K; p.group_size = G; p.zero_offset = zero_offset;
    p.stride_am = K; p.stride_ak = 1;
    if (fmt == W4A16_FMT_AWQ) { p.stride_qwk = N / 8; p.stride_qwn = 1; }
    else { p.stride_qwk = N; p.stride_qwn = 1; }
    p.stride_sk = N; p.stride_sn = 1;
    p.stride_qzk = N / 8; p.stride_qzn = 1;
    p.stride_cm = N; p.stride_cn = 1;
    p.gate = gate;
    p.gate_want = 0;
    hipError_t e = launch_strided_gemm(fmt, p, st, bf16);
    if (e != hipSuccess) return hip_fail(e, "strided gemm launch");
    return W4A16_OK;
}

}  // namespace w4a16

extern "C" {

W4A16_API int w4a16_gemm(void* stream, int fmt, const void* x, const void* qweight,
                         const void* scales, const void* qzeros, const int32_t* g_idx, void* out,
                         int32_t M, int32_t N, int32_t K, int32_t G, int32_t zero_offset) {
    return gemm_impl(stream, fmt, x, qweight, scales, qzeros, g_idx, out, M, N, K, G, zero_offset,
                     alloc_scratch_source());
}

// ------------------------------------------------------------------ act-order in group order

W4A16_API int w4a16_prepare_act_order(void* stream, int fmt, const void* qweight,
                                      const int32_t* g_idx, int32_t K, int32_t N, int32_t G,
                                      void* qweight_out, int32_t* perm_out) {
    if (fmt != W4A16_FMT_GPTQ && fmt != W4A16_FMT_GPTQ_SYM)
        return fail(W4A16_ERR_INVALID_ARG, "act-order repack takes the GPTQ formats (fmt %d)", fmt);
    if (!qweight || !g_idx || !qweight_out || !perm_out)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (K < 8 || N < 1 || G < 1 || K % 8 || K % G)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (K=%d N=%d group_size=%d)", K, N, G);
    if (K / 8 > 65535) return fail(W4A16_ERR_UNSUPPORTED, "K (%d) above 524280", K);
    if (qweight == qweight_out)
        return fail(W4A16_ERR_INVALID_ARG, "qweight_out must not alias qweight");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (stream_capturing(st))
        return fail(W4A16_ERR_UNSUPPORTED, "w4a16_prepare_act_order synchronises: not under capture");
    // the group table is read on the host (once per checkpoint): validated, then sorted
    std::vector<int32_t> gi((size_t)K), perm((size_t)K);
    hipError_t e = hipMemcpyAsync(gi.data(), g_idx, (size_t)K * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "reading g_idx");
    const int groups = K / G;
    std::vector<int32_t> start((size_t)groups + 1, 0);
    for (int k = 0; k < K; ++k) {
        if (gi[k] < 0 || gi[k] >= groups)
            return fail(W4A16_ERR_INVALID_ARG, "g_idx[%d] = %d outside [0, %d)", k, gi[k], groups);
        ++start[(size_t)gi[k] + 1];
    }
    for (int g = 0; g < groups; ++g) {
        if (start[(size_t)g + 1] != G)
            return fail(W4A16_ERR_INVALID_ARG,
                        "group %d holds %d rows; group order needs exactly group_size (%d) rows "
                        "per group", g, start[(size_t)g + 1], G);
        start[(size_t)g + 1] += start[(size_t)g];
    }
    for (int k = 0; k < K; ++k) perm[(size_t)start[(size_t)gi[k]]++] = k;   // stable in k
    e = hipMemcpyAsync(perm_out, perm.data(), (size_t)K * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "writing perm");
    e = launch_gptq_repack_rows(static_cast<const uint32_t*>(qweight), perm_out,
                                static_cast<uint32_t*>(qweight_out), K, N, st);
    // the host copy of perm must outlive the transfer: wait whatever the launch returned
    const hipError_t es = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "act-order repack launch");
    return es == hipSuccess ? W4A16_OK : hip_fail(es, "act-order repack");
}

W4A16_API int w4a16_gemm_act_order(void* stream, int fmt, const void* x, const void* qweight,
                                   const void* scales, const void* qzeros, const int32_t* perm,
                                   void* out, int32_t M, int32_t N, int32_t K, int32_t G,
                                   int32_t zero_offset) {
    if (fmt != W4A16_FMT_GPTQ && fmt != W4A16_FMT_GPTQ_SYM)
        return fail(W4A16_ERR_INVALID_ARG, "act-order GEMM takes the GPTQ formats (fmt %d)", fmt);
    int rc = check_gemm_args(fmt, x, qweight, scales, qzeros, out, M, N, K, G);
    if (!rc) rc = check_zero_offset(fmt, zero_offset);
    if (rc) return rc;
    if (!perm) return fail(W4A16_ERR_INVALID_ARG, "perm is null");
    if (!aligned(x, 16)) return fail(W4A16_ERR_INVALID_ARG, "x must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* xg = nullptr;
    rc = stream_buffer(g_gather, st, (size_t)M * K * sizeof(half_t), 0, "act-order gather buffer", &xg);
    if (rc) return rc;
    hipError_t e = launch_gather_columns(static_cast<const half_t*>(x), perm,
                                         static_cast<half_t*>(xg), M, K, st);
    if (e != hipSuccess) return hip_fail(e, "act-order gather launch");
    return gemm_impl(stream, fmt, xg, qweight, scales, qzeros, nullptr, out, M, N, K, G,
                     zero_offset, alloc_scratch_source());
}

// ------------------------------------------------------------------ prepared layout

static int check_prep_shape(int32_t K, int32_t N, int32_t G) {
    if (K < 1 || N < 1 || G < 1)
        return fail(W4A16_ERR_INVALID_ARG, "sizes must be positive (K=%d N=%d group_size=%d)", K, N, G);
    if (K % G) return fail(W4A16_ERR_INVALID_ARG, "K (%d) must be a multiple of group_size (%d)", K, G);
    if (N % 16 || K % 128 || !prep_group_ok(G) || K > PREP_MAX_K)
        return fail(W4A16_ERR_UNSUPPORTED,
                    "the prepared layout needs N %% 16 == 0, K %% 128 == 0, group_size 32, 64 or a "
                    "multiple of 128, and K <= %d (K=%d N=%d group_size=%d)", PREP_MAX_K, K, N, G);
    return W4A16_OK;
}

W4A16_API size_t w4a16_prepared_bytes(int32_t K, int32_t N, int32_t G) {
    if (K < 1 || N < 1 || G < 1 || K % G || N % 16 || K % 128 || !prep_group_ok(G) || K > PREP_MAX_K)
        return 0;
    return prep_total_bytes(K, N, G);
}

W4A16_API int w4a16_prepare_layout(void* stream, int fmt, const void* qweight, const void* scales,
                                   const void* qzeros, int32_t K, int32_t N, int32_t G,
                                   int32_t zero_offset, void* prepared, size_t prepared_bytes) {
    int rc = check_gemm_args(fmt, (void*)1, qweight, scales, qzeros, (void*)1, 1, N, K, G);
    if (!rc) rc = check_zero_offset(fmt, zero_offset);
    if (!rc) rc = check_prep_shape(K, N, G);
    if (rc) return rc;
    if (!prepared) return fail(W4A16_ERR_INVALID_ARG, "prepared is null");
    const size_t need = prep_total_bytes(K, N, G);
    if (prepared_bytes < need)
        return fail(W4A16_ERR_INVALID_ARG, "prepared buffer too small (%zu < %zu bytes)", prepared_bytes, need);
    if (!aligned(prepared, 256)) return fail(W4A16_ERR_INVALID_ARG, "prepared must be 256-byte aligned");
    const char* pb = static_cast<const char*>(prepared);
    auto overlaps = [&](const void* q, size_t n) {
        const char* c = static_cast<const char*>(q);
        return q && c < pb + need && pb < c + n;
    };
    if (overlaps(qweight, (size_t)K * N / 2) || overlaps(scales, (size_t)(K / G) * N * 2) ||
        (fmt != W4A16_FMT_GPTQ_SYM && overlaps(qzeros, (size_t)(K / G) * N / 2)))
        return fail(W4A16_ERR_INVALID_ARG, "prepared must not overlap the checkpoint tensors");
    hipError_t e = launch_prepare_layout(
        fmt, static_cast<const uint32_t*>(qweight), static_cast<const half_t*>(scales),
        fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros), prepared, K, N,
        G, zero_offset, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepare layout launch");
}

W4A16_API int w4a16_dequant_prepared(void* stream, const void* prepared, void* out, int32_t K,
                                     int32_t N, int32_t G, int transposed) {
    if (int rc = check_prep_shape(K, N, G)) return rc;
    if (!prepared || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (!aligned(prepared, 256) || !aligned(out, 16))
        return fail(W4A16_ERR_INVALID_ARG, "prepared must be 256-byte and out 16-byte aligned");
    hipError_t e = launch_prep_dequant(prepared, static_cast<half_t*>(out), K, N, G,
                                       transposed ? 1 : 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared dequant launch");
}

W4A16_API int w4a16_gemm_prepared(void* stream, const void* x, const void* prepared,
                                  const int32_t* perm, void* out, int32_t M, int32_t N, int32_t K,
                                  int32_t G) {
    if (int rc = check_prep_shape(K, N, G)) return rc;
    if (!x || !prepared || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (M < 1) return fail(W4A16_ERR_INVALID_ARG, "M (%d) must be positive", M);
    if (!aligned(x, 16) || !aligned(prepared, 256) || !aligned(out, 16) || (perm && !aligned(perm, 16)))
        return fail(W4A16_ERR_INVALID_ARG,
                    "x, out and perm must be 16-byte aligned, prepared 256-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // 2..64 rows (5..64 without act-order, or 4 where a wave takes 4 blocks, K <= 4096; below
    // that the rows GEMV is as fast or faster: AWQ M = 4 4096 -> 14336 9.13 -> 8.73 us, 14336
    // -> 4096 9.45 -> 9.80 us, M = 3 8.63 -> 8.69 us): the small-batch kernel, reading x as
    // stored (act-order: x's columns gathered by perm first) and putting it in MFMA fragment
    // order itself
    const PrepFragShape fs = prep_frag_shape(M, N, K, G);
    if (fs.ok && (perm ? M >= 2 : M >= 5 || (M == 4 && fs.bpw == 4))) {
        const void* xa = x;
        hipError_t e = hipSuccess;
        if (perm) {
            void* xg = nullptr;
            int rc = stream_buffer(g_gather, st, (size_t)M * K * sizeof(half_t), 0, "act-order gather buffer", &xg);
            if (rc) return rc;
            e = launch_gather_columns(static_cast<const half_t*>(x), perm, static_cast<half_t*>(xg), M, K, st);
            if (e != hipSuccess) return hip_fail(e, "act-order gather launch");
            xa = xg;
        }
        PrepFragParams p{};
        p.x = static_cast<const half_t*>(xa);
        p.prep = static_cast<const unsigned char*>(prepared);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G;
        p.strip_bytes = (uint32_t)prep_strip_bytes(K, G);
        e = launch_prep_frag(p, fs, st);
        return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared small-batch launch");
    }
    const void* xa = x;
    if (perm) {   // act-order checkpoint prepared in group order: x' = x[:, perm]
        void* xg = nullptr;
        int rc = stream_buffer(g_gather, st, (size_t)M * K * sizeof(half_t), 0, "act-order gather buffer", &xg);
        if (rc) return rc;
        hipError_t e = launch_gather_columns(static_cast<const half_t*>(x), perm,
                                             static_cast<half_t*>(xg), M, K, st);
        if (e != hipSuccess) return hip_fail(e, "act-order gather launch");
        xa = xg;
    }
    // M <= 8: the GEMV kernels (one workgroup per strip, no split-K)
    const PrepGemvShape gs = prep_gemv_shape(M, N, K, G);
    if (gs.ok) {
        PrepParams p{};
        p.x = static_cast<const half_t*>(xa);
        p.prep = static_cast<const unsigned char*>(prepared);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G;
        p.strip_bytes = (uint32_t)prep_strip_bytes(K, G);
        hipError_t e = launch_prep_gemv(p, gs, st);
        return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared gemv launch");
    }
    // larger M: the pipelined prefill kernel reading the prepared strips (64-row stages: the
    // group size must be a multiple of 64; 32-bit offsets into the prepared buffer)
    const int cus = device_cus();
    PrefillShape ps = prefill_shape(FMT_PREP, M, N, K, G, cus);
    const bool pre_ok = ps.ok && ps.dma && G % 64 == 0 && prep_total_bytes(K, N, G) < ((size_t)1 << 31);
    if (pre_ok) {
        PrefillParams p{};
        p.x = static_cast<const half_t*>(xa);
        p.qweight = static_cast<const uint32_t*>(prepared);
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G;
        p.ksplit = ps.ksplit;
        if (ps.ksplit > 1) {
            uint32_t* counters = nullptr;
            float* partials = nullptr;
            const size_t tiles = (size_t)ps.col_tiles * ps.row_tiles;
            if (tiles > SPLITK_MAX_TILES) {
                ps = prefill_shape(FMT_PREP, M, N, K, G, cus, 1);
                p.ksplit = 1;
            } else {
                if (int rc = get_workspace(st, (size_t)ps.ksplit * M * N * sizeof(float), &counters, &partials))
                    return rc;
                p.counters = counters;
                p.ws = partials;
            }
        }
        hipError_t e = launch_prefill(FMT_PREP, p, ps, st);
        return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared prefill launch");
    }
    // any other shape: the generic kernel, dequantising each element from the strips
    StridedParams p{};
    p.a = static_cast<const half_t*>(xa);
    p.qweight = static_cast<const uint32_t*>(prepared);
    p.c = static_cast<half_t*>(out);
    p.m = M; p.n = N; p.k = K; p.group_size = G;
    p.stride_am = K; p.stride_ak = 1;
    p.stride_qwk = (int)(prep_strip_bytes(K, G) / 4);   // words per strip
    p.stride_qwn = (int)prep_table_words(K, G);         // words of the strip's table
    p.stride_cm = N; p.stride_cn = 1;
    hipError_t e = launch_strided_gemm(FMT_PREP, p, st);
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared strided gemm launch");
}

W4A16_API int w4a16_gemm_prepared_gidx(void* stream, const void* x, const void* prepared,
                                       const int32_t* g_idx, void* out, int32_t M, int32_t N,
                                       int32_t K, int32_t G) {
    if (int rc = check_prep_shape(K, N, G)) return rc;
    if (!x || !prepared || !g_idx || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (M < 1) return fail(W4A16_ERR_INVALID_ARG, "M (%d) must be positive", M);
    if (!aligned(x, 16) || !aligned(prepared, 256) || !aligned(out, 16) || !aligned(g_idx, 16))
        return fail(W4A16_ERR_INVALID_ARG,
                    "x, out and g_idx must be 16-byte aligned, prepared 256-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // up to 64 rows (K <= 4096): the small-batch kernel with the per-workgroup (scale, zero)
    // table filled from the strips' own tables and indexed through g_idx; x read as stored
    const PrepFragShape fs = prep_frag_shape(M, N, K, G, /*act=*/true);
    if (fs.ok) {
        PrepFragParams p{};
        p.x = static_cast<const half_t*>(x);
        p.prep = static_cast<const unsigned char*>(prepared);
        p.g_idx = g_idx;
        p.out = static_cast<half_t*>(out);
        p.M = M; p.N = N; p.K = K; p.G = G;
        p.strip_bytes = (uint32_t)prep_strip_bytes(K, G);
        hipError_t e = launch_prep_frag(p, fs, st);
        return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared act-order small-batch launch");
    }
    // any other shape: the generic kernel, each element's (scale, zero) from its group's row
    // of the strip's table
    StridedParams p{};
    p.a = static_cast<const half_t*>(x);
    p.qweight = static_cast<const uint32_t*>(prepared);
    p.g_idx = g_idx;
    p.c = static_cast<half_t*>(out);
    p.m = M; p.n = N; p.k = K; p.group_size = G;
    p.stride_am = K; p.stride_ak = 1;
    p.stride_qwk = (int)(prep_strip_bytes(K, G) / 4);
    p.stride_qwn = (int)prep_table_words(K, G);
    p.stride_cm = N; p.stride_cn = 1;
    hipError_t e = launch_strided_gemm(FMT_PREP, p, st);
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "prepared act-order strided gemm launch");
}

// The reference kernels' parameter lists with arbitrary strides. A call whose tensors are
// the dense row-major layouts of the checkpoint formats (the usual case: a linear layer's
// weights and activations) is the same problem w4a16_gemm solves, and goes through its
// planner to the GEMV / small-batch / prefill kernels; anything else (transposed or padded
// operands, shapes those kernels reject) runs the generic strided kernel. Both give the
// reference's result: W16 = RNE_f16((q - z) s) with z = nibble + 1 (GPTQ) or the nibble
// (AWQ), fp32 accumulation, fp16 output.
static bool typed_dense(int fmt, const void* a, const void* qw, const void* sc, const void* qz,
                        const void* c, int32_t m, int32_t n, int32_t k, int32_t G,
                        const int32_t* st) {
    if (n % 8 || k % G || (fmt == W4A16_FMT_GPTQ && k % 8)) return false;
    const int32_t qw_k = fmt == W4A16_FMT_AWQ ? n / 8 : n;
    const bool rows_ok = (st[0] == k || m == 1) && st[1] == 1 &&      // a [m, k]
                         st[2] == qw_k && st[3] == 1 &&                // qweight
                         st[4] == n && st[5] == 1 &&                   // scales [k/G, n]
                         st[6] == n / 8 && st[7] == 1 &&               // qzeros [k/G, n/8]
                         (st[8] == n || m == 1) && st[9] == 1;         // c [m, n]
    return rows_ok && aligned(a, 16) && aligned(qw, 16) && aligned(sc, 16) && aligned(qz, 16) &&
           aligned(c, 16);
}

static int typed_common(int fmt, void* stream, const void* a, const void* qw, const void* sc,
                        const void* qz, void* c, int32_t m, int32_t n, int32_t k, int32_t G,
                        const int32_t* strides) {
    if (!a || !qw || !sc || !qz || !c)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (m < 0 || n < 0 || k < 0 || G < 1)
        return fail(W4A16_ERR_INVALID_ARG, "negative size or group_size < 1");
    if (m == 0 || n == 0) return W4A16_OK;
    if (k > 0 && typed_dense(fmt, a, qw, sc, qz, c, m, n, k, G, strides))
        return w4a16_gemm(stream, fmt, a, qw, sc, qz, nullptr, c, m, n, k, G,
                          fmt == W4A16_FMT_GPTQ ? 1 : 0);
    StridedParams p{};
    p.a = static_cast<const half_t*>(a);
    p.qweight = static_cast<const uint32_t*>(qw);
    p.scales = static_cast<const half_t*>(sc);
    p.qzeros = static_cast<const uint32_t*>(qz);
    p.g_idx = nullptr;
    p.c = static_cast<half_t*>(c);
    p.m = m; p.n = n; p.k = k; p.group_size = G;
    p.stride_am = strides[0]; p.stride_ak = strides[1];
    p.stride_qwk = strides[2]; p.stride_qwn = strides[3];
    p.stride_sk = strides[4]; p.stride_sn = strides[5];
    p.stride_qzk = strides[6]; p.stride_qzn = strides[7];
    p.stride_cm = strides[8]; p.stride_cn = strides[9];
    p.zero_offset = (fmt == W4A16_FMT_GPTQ) ? 1 : 0;
    hipError_t e = launch_strided_gemm(fmt, p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "typed gemm launch");
    return W4A16_OK;
}

W4A16_API int w4a16_typed_plan(int fmt, int32_t m, int32_t n, int32_t k, int32_t group_size,
                               const int32_t* strides, int aligned16, int* kernel) {
    if (fmt != W4A16_FMT_GPTQ && fmt != W4A16_FMT_AWQ)
        return fail(W4A16_ERR_INVALID_ARG, "typed entry points take GPTQ or AWQ (fmt %d)", fmt);
    if (!strides || !kernel) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (m < 1 || n < 1 || k < 1 || group_size < 1)
        return fail(W4A16_ERR_INVALID_ARG, "sizes must be positive");
    const void* p = aligned16 ? (const void*)(uintptr_t)256 : (const void*)(uintptr_t)2;
    *kernel = typed_dense(fmt, p, p, p, p, p, m, n, k, group_size, strides)
                  ? plan(fmt, m, n, k, group_size, false)
                  : W4A16_KERNEL_STRIDED;
    return W4A16_OK;
}

W4A16_API int w4a16_gptq_gemm_typed(void* stream, const void* a_ptr, const void* qweight_ptr,
                                    const void* scales_ptr, const void* qzeros_ptr, void* c_ptr,
                                    int32_t m_size, int32_t n_size, int32_t k_size,
                                    int32_t group_size, int32_t stride_am, int32_t stride_ak,
                                    int32_t stride_qwk, int32_t stride_qwn, int32_t stride_sk,
                                    int32_t stride_sn, int32_t stride_qzk, int32_t stride_qzn,
                                    int32_t stride_cm, int32_t stride_cn) {
    const int32_t s[10] = {stride_am, stride_ak, stride_qwk, stride_qwn, stride_sk,
                           stride_sn, stride_qzk, stride_qzn, stride_cm, stride_cn};
    return typed_common(W4A16_FMT_GPTQ, stream, a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr,
                        m_size, n_size, k_size, group_size, s);
}

W4A16_API int awq_gemm_int4_typed(void* stream, const void* a_ptr, const void* qweight_ptr,
                                  const void* scales_ptr, const void* qzeros_ptr, void* c_ptr,
                                  int32_t m_size, int32_t n_size, int32_t k_size,
                                  int32_t group_size, int32_t stride_am, int32_t stride_ak,
                                  int32_t stride_qwk, int32_t stride_qwn, int32_t stride_sk,
                                  int32_t stride_sn, int32_t stride_qzk, int32_t stride_qzn,
                                  int32_t stride_cm, int32_t stride_cn) {
    const int32_t s[10] = {stride_am, stride_ak, stride_qwk, stride_qwn, stride_sk,
                           stride_sn, stride_qzk, stride_qzn, stride_cm, stride_cn};
    return typed_common(W4A16_FMT_AWQ, stream, a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr,
                        m_size, n_size, k_size, group_size, s);
}

static int dequant_common(void* stream, int fmt, const void* qweight, const void* scales,
                          const void* qzeros, const int32_t* g_idx, void* out, int32_t K,
                          int32_t N, int32_t G, int32_t zero_offset, int transposed) {
    const bool bf16 = (fmt & W4A16_BF16) != 0;
    fmt &= ~W4A16_BF16;
    int rc = check_gemm_args(fmt, (void*)1, qweight, scales, qzeros, out, 1, N, K, G);
    if (!rc) rc = check_zero_offset(fmt, zero_offset);
    if (rc) return rc;
    if (fmt == W4A16_FMT_AWQ && !aligned(out, 16) && !transposed)
        return fail(W4A16_ERR_INVALID_ARG, "out must be 16-byte aligned");
    if (fmt != W4A16_FMT_AWQ && transposed && (!aligned(out, 16) || K % 8))
        return fail(W4A16_ERR_INVALID_ARG, "out must be 16-byte aligned");
    DequantParams p{};
    p.qweight = static_cast<const uint32_t*>(qweight);
    p.scales = static_cast<const half_t*>(scales);
    p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
    p.g_idx = g_idx;
    p.out = static_cast<half_t*>(out);
    p.K = K; p.N = N; p.G = G; p.zero_offset = zero_offset; p.transposed = transposed;
    hipError_t e = launch_dequant(fmt, p, static_cast<hipStream_t>(stream), bf16);
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return W4A16_OK;
}

W4A16_API int dequant_int4_to_fp16(void* stream, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, void* output, int32_t k_dim,
                                   int32_t n_dim, int32_t group_size, int32_t n_div_8) {
    if (n_div_8 * 8 != n_dim)
        return fail(W4A16_ERR_INVALID_ARG, "n_div_8 (%d) must equal n_dim / 8 (n_dim=%d)", n_div_8,
                    n_dim);
    return dequant_common(stream, W4A16_FMT_GPTQ, qweight, scales, qzeros, nullptr, output, k_dim,
                          n_dim, group_size, 0, 1);
}

W4A16_API int dequant_int4_sym_to_fp16(void* stream, const int32_t* qweight, const void* scales,
                                       void* output, int32_t k_dim, int32_t n_dim,
                                       int32_t group_size) {
    return dequant_common(stream, W4A16_FMT_GPTQ_SYM, qweight, scales, nullptr, nullptr, output,
                          k_dim, n_dim, group_size, 0, 1);
}

W4A16_API int w4a16_dequant(void* stream, int fmt, const void* qweight, const void* scales,
                            const void* qzeros, const int32_t* g_idx, void* out, int32_t K,
                            int32_t N, int32_t G, int32_t zero_offset, int transposed) {
    return dequant_common(stream, fmt, qweight, scales, qzeros, g_idx, out, K, N, G, zero_offset,
                          transposed ? 1 : 0);
}

// ------------------------------------------------------------------ fused MoE

static int check_moe_dims(int32_t T, int32_t E, int32_t topk) {
    if (T < 1 || E < 1 || topk < 1 || topk > E)
        return fail(W4A16_ERR_INVALID_ARG, "bad MoE sizes (T=%d E=%d topk=%d)", T, E, topk);
    if (E > 256 || topk > 8)
        return fail(W4A16_ERR_UNSUPPORTED, "MoE supports E <= 256 experts and topk <= 8");
    return W4A16_OK;
}

W4A16_API int w4a16_moe_route(void* stream, const float* logits, int32_t T, int32_t E,
                              int32_t topk, int32_t renormalize, int32_t* topk_ids,
                              float* topk_weights) {
    if (!logits || !topk_ids || !topk_weights)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (int rc = check_moe_dims(T, E, topk)) return rc;
    hipError_t e = launch_moe_route(logits, T, E, topk, renormalize, topk_ids, topk_weights,
                                    static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "moe route launch");
}

W4A16_API int w4a16_moe_align(void* stream, const int32_t* topk_ids, int32_t num_pairs, int32_t E,
                              int32_t block_m, int32_t capacity, int32_t* sorted_ids,
                              int32_t* expert_ids, int32_t* num_tokens_post_padded) {
    if (!topk_ids || !sorted_ids || !expert_ids || !num_tokens_post_padded)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (num_pairs < 1 || E < 1 || block_m < 1)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (pairs=%d E=%d block_m=%d)", num_pairs, E,
                    block_m);
    if (E > 1024) return fail(W4A16_ERR_UNSUPPORTED, "moe_align supports at most 1024 experts");
    const int64_t need = (int64_t)num_pairs + (int64_t)E * (block_m - 1);
    if (capacity < need || capacity % block_m)
        return fail(W4A16_ERR_INVALID_ARG,
                    "capacity (%d) must be a multiple of block_m and >= pairs + E*(block_m-1) = %lld",
                    capacity, (long long)need);
    hipError_t e = launch_moe_align(topk_ids, num_pairs, E, block_m, capacity, sorted_ids,
                                    expert_ids, num_tokens_post_padded,
                                    static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "moe align launch");
}

W4A16_API int w4a16_moe_gemm(void* stream, int fmt, const void* a, int32_t a_div,
                             const void* qweight, const void* scales, const void* qzeros,
                             int64_t qweight_expert_stride, int64_t scales_expert_stride,
                             int64_t qzeros_expert_stride, int32_t num_experts,
                             const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                             void* out, int32_t num_pairs, int32_t N, int32_t K, int32_t G,
                             int32_t block_m, int32_t capacity, int32_t zero_offset) {
    int rc = check_gemm_args(fmt, a, qweight, scales, qzeros, out, 1, N, K, G);
    if (!rc) rc = check_zero_offset(fmt, zero_offset);
    if (rc) return rc;
    if (!sorted_ids || !expert_ids || !num_tokens_post_padded)
        return fail(W4A16_ERR_INVALID_ARG, "null routing pointer");
    if (a_div < 1 || num_pairs < 1 || capacity < 1 || block_m < 1 || capacity % block_m ||
        num_experts < 1)
        return fail(W4A16_ERR_INVALID_ARG, "bad grouped-GEMM sizes");
    if (!moe_gemm_supported(N, K, G, block_m))
        return fail(W4A16_ERR_UNSUPPORTED,
                    "grouped GEMM needs N %% 256 == 0, K %% 64 == 0, group_size %% 8 == 0 and "
                    "block_m in {64, 128} (N=%d K=%d G=%d block_m=%d)", N, K, G, block_m);
    if (!aligned(a, 16) || !aligned(qweight, 16) || !aligned(scales, 16) || !aligned(out, 16))
        return fail(W4A16_ERR_INVALID_ARG, "tensors must be 16-byte aligned");
    PrefillParams p{};
    p.x = static_cast<const half_t*>(a);
    p.qweight = static_cast<const uint32_t*>(qweight);
    p.scales = static_cast<const half_t*>(scales);
    p.qzeros = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : static_cast<const uint32_t*>(qzeros);
    p.out = static_cast<half_t*>(out);
    p.M = capacity; p.N = N; p.K = K; p.G = G; p.zero_offset = zero_offset;
    p.sorted_ids = sorted_ids; p.expert_ids = expert_ids;
    p.num_post_padded = num_tokens_post_padded;
    p.num_pairs = num_pairs; p.a_div = a_div; p.num_experts = num_experts;
    p.qweight_stride = qweight_expert_stride; p.scales_stride = scales_expert_stride;
    p.qzeros_stride = qzeros_expert_stride;
    hipError_t e = launch_moe_gemm(fmt, p, block_m, capacity / block_m,
                                   static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "moe gemm launch");
}

W4A16_API int fused_silu_mul_interleaved_f16(void* stream, const void* gate_up, void* out,
                                             int32_t inter, int32_t total) {
    if (!gate_up || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (inter < 1 || total < 0)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (inter=%d total=%d)", inter, total);
    if (total == 0) return W4A16_OK;
    hipError_t e = launch_silu_mul(static_cast<const half_t*>(gate_up), static_cast<half_t*>(out),
                                   inter, total, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "silu_mul launch");
}

W4A16_API int fused_silu_mul_interleaved_f32(void* stream, const float* gate_up, float* out,
                                             int32_t inter, int32_t total) {
    if (!gate_up || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (inter < 1 || total < 0)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (inter=%d total=%d)", inter, total);
    if (total == 0) return W4A16_OK;
    hipError_t e = launch_silu_mul_f32(gate_up, out, inter, total, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "silu_mul_f32 launch");
}

W4A16_API int w4a16_moe_sum(void* stream, const void* y_pairs, const float* topk_weights,
                            void* out, int32_t T, int32_t topk, int32_t K) {
    if (!y_pairs || !topk_weights || !out) return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (T < 1 || topk < 1 || K < 8 || K % 8)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (T=%d topk=%d K=%d)", T, topk, K);
    hipError_t e = launch_moe_sum(static_cast<const half_t*>(y_pairs), topk_weights,
                                  static_cast<half_t*>(out), T, topk, K,
                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : hip_fail(e, "moe sum launch");
}

namespace {
struct MoeLayout {
    size_t ids, weights, sorted, experts, npp, tiles, ntiles, h, a, yp, part, ctr, total;
    int32_t capacity, max_tiles, n_ctr;
};
// The down projection may split its K (= I) in two (moe_tiles): fp32 partials for every
// pair and a counter per tile. Reserved whenever the shape allows the split.
bool moe_down_may_split(int32_t K, int32_t I) { return K % 256 == 0 && I % 128 == 0 && I / 128 >= 64; }
size_t up256(size_t v) { return (v + 255) / 256 * 256; }
MoeLayout moe_layout(int32_t T, int32_t E, int32_t topk, int32_t I, int32_t K, int32_t block_m) {
    MoeLayout L{};
    const int64_t P = (int64_t)T * topk;
    const int64_t cap = (P + (int64_t)E * (block_m - 1) + block_m - 1) / block_m * block_m;
    L.capacity = (int32_t)cap;
    size_t off = 0;
    L.ids = off; off = up256(off + P * 4);
    L.weights = off; off = up256(off + P * 4);
    L.sorted = off; off = up256(off + cap * 4);
    L.experts = off; off = up256(off + cap / block_m * 4);
    L.npp = off; off = up256(off + 4);
    L.max_tiles = moe_max_tiles((int)P, E, 64);   // bound for every tile height >= 64
    L.tiles = off; off = up256(off + (size_t)L.max_tiles * 16);
    L.ntiles = off; off = up256(off + 4);
    L.h = off; off = up256(off + (size_t)P * 2 * I * 2);
    L.a = off; off = up256(off + (size_t)P * I * 2);
    L.yp = off; off = up256(off + (size_t)P * K * 2);
    L.n_ctr = 0;
    L.part = L.ctr = off;
    if (moe_down_may_split(K, I)) {
        L.part = off; off = up256(off + (size_t)2 * P * K * 4);
        L.n_ctr = L.max_tiles * (K / 256);
        L.ctr = off; off = up256(off + (size_t)L.n_ctr * FLAG_STRIDE * 4);
    }
    L.total = off;
    return L;
}

// Expert-tile shape of the fused layer's grouped GEMMs. Tile height: the smallest of 64,
// 128, 192, 256 rows holding 1.25x the mean rows per expert, so that one tile usually covers
// all of an expert's tokens and its weights are dequantised once per column tile. Tile
// width: the fewest rounds of workgroups over the CUs times the width (ties to the wider
// tile), for the tile count a balanced routing gives; 64-row tiles come 256 wide only.
struct MoeTiles { int bm, bn13, bn2, ks2; };
int moe_tile_bn(int N, int bm, int est_tiles, int cus) {
    if (bm == 64) return 256;
    int best = 0;
    long long best_cost = 0;
    for (int bn : {256, 224, 128}) {
        if (N % bn) continue;
        const long long wgs = (long long)est_tiles * (N / bn);
        const long long cost = (wgs + cus - 1) / cus * bn;
        if (!best || cost < best_cost) { best = bn; best_cost = cost; }
    }
    return best;
}
MoeTiles moe_tiles(int P, int E, int K, int I, int cus) {
    const double want = 1.25 * P / E;
    MoeTiles t{};
    t.bm = want <= 64 ? 64 : want <= 128 ? 128 : want <= 192 ? 192 : 256;
    const int per_expert = (int)((P / E + t.bm - 1) / t.bm);
    const int est = E * (per_expert > 0 ? per_expert : 1);
    t.bn13 = moe_tile_bn(2 * I, t.bm, est, cus);
    t.bn2 = moe_tile_bn(K, t.bm, est, cus);
    // down projection with 128-wide tiles and a long K: 256-wide tiles with K split in two
    // (as the dense prefill does; config 4: 16 x 8 x 2 = 256 workgroups)
    t.ks2 = 1;
    if (t.bn2 == 128 && t.bm > 64 && moe_down_may_split(K, I) &&
        (long long)est * (K / 256) * 2 <= cus) {
        t.bn2 = 256;
        t.ks2 = 2;
    }
    return t;
}
}  // namespace

W4A16_API size_t w4a16_fused_moe_workspace_size(int32_t T, int32_t E, int32_t topk, int32_t I,
                                                int32_t K, int32_t block_m) {
    if (T < 1 || E < 1 || topk < 1 || I < 1 || K < 1 || block_m < 1) return 0;
    return moe_layout(T, E, topk, I, K, block_m).total;
}

// The expert-tile layer after routing: align into expert tiles, gate/up GEMM, silu * mul,
// down GEMM (K split as moe_tiles chose), weighted sum. Weights in a checkpoint format or in
// the prepared layout (fmt FMT_PREP: the q pointers are stacked prepared buffers, the scale and
// zero pointers unused).
struct MoeWeights {
    int fmt;
    const void *w13q, *w13s, *w13z, *w2q, *w2s, *w2z;
    int64_t q13, s13, z13, q2, s2, z2;   // per-expert strides in elements
    int32_t zero_offset;
};
static int fused_moe_tiles(void* stream, const MoeWeights& W, const void* x, int32_t T, int32_t K,
                           int32_t I, int32_t E, int32_t topk, int32_t G, int32_t block_m,
                           const MoeLayout& L, const MoeTiles& mt, char* ws, void* out) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto* ids = reinterpret_cast<int32_t*>(ws + L.ids);
    auto* wts = reinterpret_cast<float*>(ws + L.weights);
    auto* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
    auto* experts = reinterpret_cast<int32_t*>(ws + L.experts);
    auto* npp = reinterpret_cast<int32_t*>(ws + L.npp);
    auto* tiles = reinterpret_cast<int32_t*>(ws + L.tiles);
    auto* ntiles = reinterpret_cast<int32_t*>(ws + L.ntiles);
    auto* ctr = reinterpret_cast<uint32_t*>(ws + L.ctr);
    void* h = ws + L.h;
    void* a = ws + L.a;
    void* yp = ws + L.yp;
    const int32_t P = T * topk;
    const int64_t n13 = 2 * (int64_t)I;
    hipError_t e = launch_moe_align(ids, P, E, block_m, L.capacity, sorted, experts, npp, st,
                                    mt.bm, tiles, ntiles, ctr, mt.ks2 > 1 ? L.n_ctr : 0);
    if (e != hipSuccess) return hip_fail(e, "moe align launch");
    const int max_tiles = moe_max_tiles(P, E, mt.bm);
    PrefillParams p{};
    p.sorted_ids = sorted; p.expert_ids = experts; p.num_post_padded = npp;
    p.tiles = tiles; p.num_tiles = ntiles;
    p.num_pairs = P; p.G = G; p.zero_offset = W.zero_offset; p.M = L.capacity; p.num_experts = E;
    // gate/up: h[p] = x[p / topk] @ W13[e]
    p.x = static_cast<const half_t*>(x);
    p.qweight = static_cast<const uint32_t*>(W.w13q);
    p.scales = static_cast<const half_t*>(W.w13s);
    p.qzeros = static_cast<const uint32_t*>(W.w13z);
    p.out = static_cast<half_t*>(h);
    p.N = (int)n13; p.K = K; p.a_div = topk;
    p.qweight_stride = W.q13; p.scales_stride = W.s13; p.qzeros_stride = W.z13;
    e = launch_moe_gemm_tiles(W.fmt, p, mt.bm, mt.bn13, max_tiles, st);
    if (e != hipSuccess) return hip_fail(e, "moe gemm launch");
    int rc = fused_silu_mul_interleaved_f16(stream, h, a, I, P * I);
    if (rc) return rc;
    // down: yp[p] = a[p] @ W2[e]
    p.x = static_cast<const half_t*>(a);
    p.qweight = static_cast<const uint32_t*>(W.w2q);
    p.scales = static_cast<const half_t*>(W.w2s);
    p.qzeros = static_cast<const uint32_t*>(W.w2z);
    p.out = static_cast<half_t*>(yp);
    p.N = K; p.K = I; p.a_div = 1;
    p.qweight_stride = W.q2; p.scales_stride = W.s2; p.qzeros_stride = W.z2;
    if (mt.ks2 > 1) {
        p.ksplit = mt.ks2;
        p.ws = reinterpret_cast<float*>(ws + L.part);
        p.counters = ctr;
    }
    e = launch_moe_gemm_tiles(W.fmt, p, mt.bm, mt.bn2, max_tiles, st);
    if (e != hipSuccess) return hip_fail(e, "moe gemm launch");
    return w4a16_moe_sum(stream, yp, wts, out, T, topk, K);
}

W4A16_API int w4a16_fused_moe_prepared(void* stream, const void* x, const float* router_logits,
                                       int32_t T, int32_t K, int32_t I, int32_t E, int32_t topk,
                                       int32_t renormalize, const void* w13_prepared,
                                       const void* w2_prepared, int32_t G, int32_t block_m,
                                       void* workspace, size_t workspace_bytes, void* out) {
    if (!x || !router_logits || !w13_prepared || !w2_prepared || !workspace || !out)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (int rc = check_moe_dims(T, E, topk)) return rc;
    if (I < 1 || K < 1 || block_m < 1 || G < 1)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (K=%d I=%d block_m=%d group_size=%d)", K, I, block_m, G);
    if (int rc = check_prep_shape(K, 2 * I, G)) return rc;
    if (int rc = check_prep_shape(I, K, G)) return rc;
    const MoeLayout L = moe_layout(T, E, topk, I, K, block_m);
    if (workspace_bytes < L.total)
        return fail(W4A16_ERR_INVALID_ARG, "workspace too small (%zu < %zu bytes)", workspace_bytes,
                    L.total);
    if (!aligned(workspace, 256) || !aligned(w13_prepared, 256) || !aligned(w2_prepared, 256) || !aligned(x, 16))
        return fail(W4A16_ERR_INVALID_ARG,
                    "workspace and prepared buffers must be 256-byte aligned, x 16-byte aligned");
    const int32_t P = T * topk;
    const MoeTiles mt = moe_tiles(P, E, K, I, device_cus());
    const size_t b13 = prep_total_bytes(K, 2 * I, G), b2 = prep_total_bytes(I, K, G);
    if (G % 64 || !mt.bn13 || !mt.bn2 || !moe_tiles_supported(2 * I, K, G, T, mt.bn13) ||
        !moe_tiles_supported(K, I, G, P, mt.bn2) || b13 >= ((size_t)1 << 31) || b2 >= ((size_t)1 << 31))
        return fail(W4A16_ERR_UNSUPPORTED,
                    "prepared fused MoE needs the expert-tile kernels: group_size %% 64 == 0, 2I and K "
                    "multiples of the tile widths, each expert's prepared matrix under 2 GiB "
                    "(K=%d I=%d group_size=%d)", K, I, G);
    int rc = w4a16_moe_route(stream, router_logits, T, E, topk, renormalize,
                             reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + L.ids),
                             reinterpret_cast<float*>(static_cast<char*>(workspace) + L.weights));
    if (rc) return rc;
    MoeWeights W{};
    W.fmt = FMT_PREP;
    W.w13q = w13_prepared; W.w2q = w2_prepared;
    W.q13 = (int64_t)(b13 / 4); W.q2 = (int64_t)(b2 / 4);
    return fused_moe_tiles(stream, W, x, T, K, I, E, topk, G, block_m, L, mt, static_cast<char*>(workspace), out);
}

W4A16_API int w4a16_fused_moe(void* stream, int fmt, const void* x, const float* router_logits,
                              int32_t T, int32_t K, int32_t I, int32_t E, int32_t topk,
                              int32_t renormalize, const void* w13_qweight, const void* w13_scales,
                              const void* w13_qzeros, const void* w2_qweight,
                              const void* w2_scales, const void* w2_qzeros, int32_t G,
                              int32_t block_m, int32_t zero_offset, void* workspace,
                              size_t workspace_bytes, void* out) {
    if (!x || !router_logits || !workspace || !out)
        return fail(W4A16_ERR_INVALID_ARG, "null pointer argument");
    if (int rc = check_moe_dims(T, E, topk)) return rc;
    if (I < 1 || K < 1 || block_m < 1)
        return fail(W4A16_ERR_INVALID_ARG, "bad sizes (K=%d I=%d block_m=%d)", K, I, block_m);
    const MoeLayout L = moe_layout(T, E, topk, I, K, block_m);
    if (workspace_bytes < L.total)
        return fail(W4A16_ERR_INVALID_ARG, "workspace too small (%zu < %zu bytes)", workspace_bytes,
                    L.total);
    if (!aligned(workspace, 256)) return fail(W4A16_ERR_INVALID_ARG, "workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    auto* ids = reinterpret_cast<int32_t*>(ws + L.ids);
    auto* wts = reinterpret_cast<float*>(ws + L.weights);
    auto* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
    auto* experts = reinterpret_cast<int32_t*>(ws + L.experts);
    auto* npp = reinterpret_cast<int32_t*>(ws + L.npp);
    void* h = ws + L.h;
    void* a = ws + L.a;
    void* yp = ws + L.yp;
    const int32_t P = T * topk;
    int rc = w4a16_moe_route(stream, router_logits, T, E, topk, renormalize, ids, wts);
    if (rc) return rc;
    // Expert tiles (one tile per expert's rows, whatever block_m padded them to) when both
    // GEMMs take the pipelined kernel; else the grouped GEMM over block_m blocks.
    const MoeTiles mt = moe_tiles(P, E, K, I, device_cus());
    const int64_t n13 = 2 * (int64_t)I;
    if (n13 <= INT32_MAX && mt.bn13 && mt.bn2 && moe_tiles_supported((int)n13, K, G, T, mt.bn13) &&
        moe_tiles_supported(K, I, G, P, mt.bn2)) {
        if (int e = check_gemm_args(fmt, x, w13_qweight, w13_scales, w13_qzeros, h, 1, (int)n13, K, G))
            return e;
        if (int e = check_gemm_args(fmt, a, w2_qweight, w2_scales, w2_qzeros, yp, 1, K, I, G))
            return e;
        if (int e = check_zero_offset(fmt, zero_offset)) return e;
        if (!aligned(x, 16) || !aligned(w13_qweight, 16) || !aligned(w13_scales, 16) ||
            !aligned(w2_qweight, 16) || !aligned(w2_scales, 16))
            return fail(W4A16_ERR_INVALID_ARG, "tensors must be 16-byte aligned");
        MoeWeights W{};
        W.fmt = fmt;
        W.w13q = w13_qweight; W.w13s = w13_scales;
        W.w13z = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : w13_qzeros;
        W.w2q = w2_qweight; W.w2s = w2_scales; W.w2z = fmt == W4A16_FMT_GPTQ_SYM ? nullptr : w2_qzeros;
        W.q13 = (int64_t)K * n13 / 8; W.s13 = (int64_t)(K / G) * n13; W.z13 = (int64_t)(K / G) * n13 / 8;
        W.q2 = (int64_t)I * K / 8; W.s2 = (int64_t)(I / G) * K; W.z2 = (int64_t)(I / G) * K / 8;
        W.zero_offset = zero_offset;
        return fused_moe_tiles(stream, W, x, T, K, I, E, topk, G, block_m, L, mt, ws, out);
    }
    rc = w4a16_moe_align(stream, ids, P, E, block_m, L.capacity, sorted, experts, npp);
    if (!rc) {
        rc = w4a16_moe_gemm(stream, fmt, x, topk, w13_qweight, w13_scales, w13_qzeros,
                            (int64_t)K * n13 / 8, (int64_t)(K / G) * n13, (int64_t)(K / G) * n13 / 8, E,
                            sorted, experts, npp, h, P, (int32_t)n13, K, G, block_m, L.capacity,
                            zero_offset);
    }
    if (!rc) rc = fused_silu_mul_interleaved_f16(stream, h, a, I, P * I);
    if (!rc)
        rc = w4a16_moe_gemm(stream, fmt, a, 1, w2_qweight, w2_scales, w2_qzeros,
                            (int64_t)I * K / 8, (int64_t)(I / G) * K, (int64_t)(I / G) * K / 8, E,
                            sorted, experts, npp, yp, P, K, I, G, block_m, L.capacity, zero_offset);
    if (!rc) rc = w4a16_moe_sum(stream, yp, wts, out, T, topk, K);
    return rc;
}

}  // extern "C"
