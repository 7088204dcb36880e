// HIP backend for the reference's DeviceRuntime trait (crates/triton-runtime/src/lib.rs:64-85):
// load a gfx950 code object with hipModuleLoadData, look kernels up by name and launch them
// with KernelArg-style arguments packed into one parameter buffer at natural alignment
// (the convention cudarc's launch builder follows in crates/triton-runtime/examples/
// run_vec_add.rs:105-117). Also the alloc / copy / stream / event calls that the
// reference's examples take from cudarc.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/w4a16.h"

namespace w4a16 {
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
}  // namespace w4a16
using w4a16::fail;

struct hiprt_ctx {
    int device;
};

struct hiprt_module {
    hiprt_ctx* ctx;
    hipModule_t module;
    bool planned;   // the library's typed code object (w4a16_typed_module_marker present)
    mutable std::mutex mu;
    mutable std::unordered_map<std::string, hipFunction_t> fns;
};

static int dev_fail(hipError_t e, const char* what) { return w4a16::hip_fail(e, what); }

static int set_device(const hiprt_ctx* ctx) {
    hipError_t e = hipSetDevice(ctx->device);
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipSetDevice");
}

extern "C" {

W4A16_API int hiprt_create(int32_t device, hiprt_ctx** out) {
    if (!out) return fail(W4A16_ERR_INVALID_ARG, "out is null");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(W4A16_ERR_BACKEND_DISABLED, "backend `hip` has no usable device (%s)",
                    hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(W4A16_ERR_INVALID_ARG, "device %d out of range (%d devices)", device, count);
    hiprt_ctx* c = new hiprt_ctx{device};
    if (int rc = set_device(c)) { delete c; return rc; }
    *out = c;
    return W4A16_OK;
}

W4A16_API int hiprt_destroy(hiprt_ctx* ctx) {
    if (!ctx) return fail(W4A16_ERR_INVALID_ARG, "ctx is null");
    delete ctx;
    return W4A16_OK;
}

W4A16_API int hiprt_module_load(hiprt_ctx* ctx, const void* binary, size_t size,
                                hiprt_module** out) {
    if (!ctx || !binary || !out || size < 4)
        return fail(W4A16_ERR_INVALID_ARG, "null ctx/binary/out or empty binary");
    *out = nullptr;
    // A code object is an ELF file; reject anything else before handing it to the runtime.
    if (std::memcmp(binary, "\x7f" "ELF", 4) != 0)
        return fail(W4A16_ERR_MODULE_LOAD, "module load failed: not an ELF code object");
    if (int rc = set_device(ctx)) return rc;
    hipModule_t m = nullptr;
    hipError_t e = hipModuleLoadData(&m, binary);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // do not leave the failure for a later launch to report
        return fail(W4A16_ERR_MODULE_LOAD, "module load failed: %s", hipGetErrorString(e));
    }
    hiprt_module* mod = new hiprt_module();
    mod->ctx = ctx;
    mod->module = m;
    hipDeviceptr_t marker = nullptr;
    size_t marker_size = 0;
    mod->planned = hipModuleGetGlobal(&marker, &marker_size, m, "w4a16_typed_module_marker") == hipSuccess &&
                   marker_size == sizeof(uint32_t);
    (void)hipGetLastError();
    *out = mod;
    return W4A16_OK;
}

W4A16_API int hiprt_module_unload(hiprt_module* module) {
    if (!module) return fail(W4A16_ERR_INVALID_ARG, "module is null");
    hipError_t e = hipModuleUnload(module->module);
    delete module;
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipModuleUnload");
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// A launch of w4a16_gptq_gemm_typed or awq_gemm_int4_typed from the library's own code object
// that follows its launch contract (the reference's 19 arguments, optionally the two scratch
// pointers, grid (cdiv(m, 64), cdiv(n, 64), 1), 256 threads, no dynamic LDS) computes the
// same function as the C-ABI entry of the same name, which plans the kernel for the shape
// (GEMV, small-batch, prefill; the generic kernel for other strides): that entry runs it, so
// that DeviceRuntime::launch by name gets the planned kernels. Returns -1 when the launch does
// not match (it then goes to the module's kernel as given).
static int launch_planned(const char* name, const uint32_t grid[3], const uint32_t block[3],
                          uint32_t shared_mem_bytes, void* stream, const hiprt_arg* args, size_t nargs) {
    const bool gptq = std::strcmp(name, "w4a16_gptq_gemm_typed") == 0;
    if (!gptq && std::strcmp(name, "awq_gemm_int4_typed") != 0) return -1;
    if (nargs != 19 && nargs != 21) return -1;
    for (size_t i = 0; i < nargs; ++i) {
        const bool ptr = i < 5 || i >= 19;
        if (ptr ? args[i].kind != HIPRT_ARG_DEVICE_PTR
                : args[i].kind != HIPRT_ARG_I32 && args[i].kind != HIPRT_ARG_U32)
            return -1;
    }
    int32_t v[14];
    for (int i = 0; i < 14; ++i) v[i] = args[5 + i].kind == HIPRT_ARG_I32 ? args[5 + i].v.i32 : (int32_t)args[5 + i].v.u32;
    const int64_t m = v[0], n = v[1];
    if (m < 1 || n < 1 || grid[0] != (uint64_t)(m + 63) / 64 || grid[1] != (uint64_t)(n + 63) / 64 || grid[2] != 1 ||
        block[0] != 256 || block[1] != 1 || block[2] != 1 || shared_mem_bytes != 0)
        return -1;
    const void* p[5];
    for (int i = 0; i < 5; ++i) p[i] = reinterpret_cast<const void*>(args[i].v.device_ptr);
    return (gptq ? w4a16_gptq_gemm_typed : awq_gemm_int4_typed)(
        stream, p[0], p[1], p[2], p[3], const_cast<void*>(p[4]), v[0], v[1], v[2], v[3], v[4], v[5],
        v[6], v[7], v[8], v[9], v[10], v[11], v[12], v[13]);
}

W4A16_API int hiprt_launch(hiprt_ctx* ctx, const hiprt_module* module, const char* kernel_name,
                           const uint32_t grid[3], const uint32_t block[3],
                           uint32_t shared_mem_bytes, void* stream, const hiprt_arg* args,
                           size_t nargs) {
    if (!ctx || !module || !kernel_name || !grid || !block || (nargs && !args))
        return fail(W4A16_ERR_INVALID_ARG, "null argument to hiprt_launch");
    for (int i = 0; i < 3; ++i)
        if (grid[i] == 0 || block[i] == 0)
            return fail(W4A16_ERR_LAUNCH_CONFIG, "invalid launch config: zero grid/block dim");
    if ((uint64_t)block[0] * block[1] * block[2] > 1024)
        return fail(W4A16_ERR_LAUNCH_CONFIG, "invalid launch config: block has more than 1024 threads");
    if (shared_mem_bytes > 160 * 1024)
        return fail(W4A16_ERR_LAUNCH_CONFIG, "invalid launch config: %u bytes of LDS exceeds 160 KiB",
                    shared_mem_bytes);

    if (module->planned) {
        if (int rc = set_device(ctx)) return rc;
        const int rc = launch_planned(kernel_name, grid, block, shared_mem_bytes, stream, args, nargs);
        if (rc != -1) return rc;
    }

    // pack KernelArg values at natural alignment
    std::vector<unsigned char> buf;
    buf.reserve(256);
    auto put = [&](const void* src, size_t n, size_t al) {
        buf.resize(align_up(buf.size(), al));
        const size_t off = buf.size();
        buf.resize(off + n);
        std::memcpy(buf.data() + off, src, n);
    };
    for (size_t i = 0; i < nargs; ++i) {
        const hiprt_arg& a = args[i];
        switch (a.kind) {
            case HIPRT_ARG_I32: put(&a.v.i32, 4, 4); break;
            case HIPRT_ARG_U32: put(&a.v.u32, 4, 4); break;
            case HIPRT_ARG_F32: put(&a.v.f32, 4, 4); break;
            case HIPRT_ARG_I64: put(&a.v.i64, 8, 8); break;
            case HIPRT_ARG_DEVICE_PTR: put(&a.v.device_ptr, 8, 8); break;
            case HIPRT_ARG_BYTES:
                if (!a.v.bytes && a.size) return fail(W4A16_ERR_INVALID_ARG, "arg %zu: null bytes", i);
                put(a.v.bytes, a.size, 8);
                break;
            default:
                return fail(W4A16_ERR_INVALID_ARG, "arg %zu: unknown kind %d", i, a.kind);
        }
    }

    hipFunction_t fn = nullptr;
    {
        std::lock_guard<std::mutex> lk(module->mu);
        auto it = module->fns.find(kernel_name);
        if (it != module->fns.end()) {
            fn = it->second;
        } else {
            hipError_t e = hipModuleGetFunction(&fn, module->module, kernel_name);
            if (e != hipSuccess || !fn) {
                (void)hipGetLastError();
                return fail(W4A16_ERR_NOT_FOUND, "kernel `%s` not found in module: %s", kernel_name,
                            hipGetErrorString(e));
            }
            module->fns.emplace(kernel_name, fn);
        }
    }
    if (int rc = set_device(ctx)) return rc;
    size_t size = buf.size();
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, buf.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                   HIP_LAUNCH_PARAM_END};
    hipError_t e = hipModuleLaunchKernel(fn, grid[0], grid[1], grid[2], block[0], block[1],
                                         block[2], shared_mem_bytes,
                                         static_cast<hipStream_t>(stream), nullptr, cfg);
    if (e != hipSuccess) return dev_fail(e, "hipModuleLaunchKernel");
    return W4A16_OK;
}

W4A16_API int hiprt_stream_create(hiprt_ctx* ctx, void** stream) {
    if (!ctx || !stream) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    if (int rc = set_device(ctx)) return rc;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return dev_fail(e, "hipStreamCreate");
    *stream = s;
    return W4A16_OK;
}

W4A16_API int hiprt_stream_destroy(void* stream) {
    if (!stream) return fail(W4A16_ERR_INVALID_ARG, "stream is null");
    hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipStreamDestroy");
}

W4A16_API int hiprt_stream_synchronize(void* stream) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipStreamSynchronize");
}

W4A16_API int hiprt_malloc(hiprt_ctx* ctx, size_t bytes, uint64_t* device_ptr) {
    if (!ctx || !device_ptr) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    if (int rc = set_device(ctx)) return rc;
    void* p = nullptr;
    // at least one byte, as the reference's examples do for the scratch slots
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) return dev_fail(e, "hipMalloc");
    *device_ptr = reinterpret_cast<uint64_t>(p);
    return W4A16_OK;
}

W4A16_API int hiprt_free(hiprt_ctx* ctx, uint64_t device_ptr) {
    if (!ctx) return fail(W4A16_ERR_INVALID_ARG, "ctx is null");
    if (int rc = set_device(ctx)) return rc;
    hipError_t e = hipFree(reinterpret_cast<void*>(device_ptr));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipFree");
}

W4A16_API int hiprt_memcpy_htod_async(uint64_t dst, const void* src, size_t bytes, void* stream) {
    if (!dst || (!src && bytes)) return fail(W4A16_ERR_INVALID_ARG, "null pointer");
    hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice,
                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipMemcpyAsync(HtoD)");
}

W4A16_API int hiprt_memcpy_dtoh_async(void* dst, uint64_t src, size_t bytes, void* stream) {
    if (!src || (!dst && bytes)) return fail(W4A16_ERR_INVALID_ARG, "null pointer");
    hipError_t e = hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), bytes,
                                  hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipMemcpyAsync(DtoH)");
}

W4A16_API int hiprt_memset_async(uint64_t dst, int value, size_t bytes, void* stream) {
    if (!dst) return fail(W4A16_ERR_INVALID_ARG, "null pointer");
    hipError_t e = hipMemsetAsync(reinterpret_cast<void*>(dst), value, bytes,
                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipMemsetAsync");
}

W4A16_API int hiprt_event_create(void** event) {
    if (!event) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return dev_fail(e, "hipEventCreate");
    *event = ev;
    return W4A16_OK;
}

W4A16_API int hiprt_event_destroy(void* event) {
    if (!event) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipEventDestroy");
}

W4A16_API int hiprt_event_record(void* event, void* stream) {
    if (!event) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipEventRecord");
}

W4A16_API int hiprt_event_synchronize(void* event) {
    if (!event) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(event));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipEventSynchronize");
}

W4A16_API int hiprt_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (!start || !stop || !ms) return fail(W4A16_ERR_INVALID_ARG, "null argument");
    hipError_t e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                       static_cast<hipEvent_t>(stop));
    return e == hipSuccess ? W4A16_OK : dev_fail(e, "hipEventElapsedTime");
}

}  // extern "C"
