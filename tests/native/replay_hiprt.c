/* Replays, through the C ABI, the hiprt_* call sequence that the Rust DeviceRuntime backend
 * (rust/triton-runtime-hip/src/lib.rs) issues for one reference-style kernel launch:
 *   HipRuntime::new        hiprt_create, w4a16_init
 *   load_module            hiprt_module_load (code object bytes borrowed for the call)
 *   create_stream          hiprt_stream_create
 *   malloc / copy_htod     hiprt_malloc, hiprt_memcpy_htod_async
 *   launch                 hiprt_launch(name, grid, block, shmem, stream, KernelArg[] as
 *                          hiprt_arg[] in the same order)
 *   synchronize / dtoh     hiprt_stream_synchronize, hiprt_memcpy_dtoh_async
 *   drop                   hiprt_free, hiprt_stream_destroy, hiprt_module_unload, hiprt_destroy
 * The launch is awq_gemm_int4_typed of w4a16_typed.hsaco with the reference's 19 parameters
 * (awq_gemm_int4_typed.rs:96-114, dense strides) and Triton's two trailing scratch pointers.
 *
 * usage: replay_hiprt <code object> <input file> <output file>
 * input:  int32 M, N, K, G; then x fp16 [M, K], qweight i32 [K, N/8], scales fp16 [K/G, N],
 *         qzeros i32 [K/G, N/8] (raw little-endian); output: fp16 [M, N]. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "w4a16.h"

static int die(const char* what, int rc) {
    fprintf(stderr, "%s failed (%d): %s\n", what, rc, w4a16_last_error());
    return 1;
}

static void* slurp(const char* path, size_t* n) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    void* buf = malloc((size_t)sz);
    if (buf && fread(buf, 1, (size_t)sz, f) != (size_t)sz) { free(buf); buf = NULL; }
    fclose(f);
    *n = (size_t)sz;
    return buf;
}

static hiprt_arg ptr_arg(uint64_t p) { hiprt_arg a = {HIPRT_ARG_DEVICE_PTR, 0, {.device_ptr = p}}; return a; }
static hiprt_arg i32_arg(int32_t v) { hiprt_arg a = {HIPRT_ARG_I32, 0, {.i32 = v}}; return a; }

int main(int argc, char** argv) {
    if (argc != 4) { fprintf(stderr, "usage: %s <hsaco> <input> <output>\n", argv[0]); return 2; }
    size_t co_size = 0, in_size = 0;
    void* co = slurp(argv[1], &co_size);
    unsigned char* in = slurp(argv[2], &in_size);
    if (!co || !in || in_size < 16) { fprintf(stderr, "cannot read inputs\n"); return 2; }
    const int32_t* hdr = (const int32_t*)in;
    const int32_t M = hdr[0], N = hdr[1], K = hdr[2], G = hdr[3];
    const size_t bx = (size_t)M * K * 2, bq = (size_t)K * N / 2, bs = (size_t)K / G * N * 2,
                 bz = (size_t)K / G * N / 2, by = (size_t)M * N * 2;
    if (in_size != 16 + bx + bq + bs + bz) { fprintf(stderr, "input size mismatch\n"); return 2; }
    const unsigned char* src = in + 16;

    hiprt_ctx* ctx = NULL;
    int rc;
    if ((rc = hiprt_create(0, &ctx))) return die("hiprt_create", rc);
    if ((rc = w4a16_init(0))) return die("w4a16_init", rc);
    hiprt_module* mod = NULL;
    if ((rc = hiprt_module_load(ctx, co, co_size, &mod))) return die("hiprt_module_load", rc);
    free(co);   /* borrowed for the call only */
    void* stream = NULL;
    if ((rc = hiprt_stream_create(ctx, &stream))) return die("hiprt_stream_create", rc);
    uint64_t dx, dq, ds, dz, dy, scratch;
    if ((rc = hiprt_malloc(ctx, bx, &dx)) || (rc = hiprt_malloc(ctx, bq, &dq)) ||
        (rc = hiprt_malloc(ctx, bs, &ds)) || (rc = hiprt_malloc(ctx, bz, &dz)) ||
        (rc = hiprt_malloc(ctx, by, &dy)) || (rc = hiprt_malloc(ctx, 1, &scratch)))
        return die("hiprt_malloc", rc);
    if ((rc = hiprt_memcpy_htod_async(dx, src, bx, stream)) ||
        (rc = hiprt_memcpy_htod_async(dq, src + bx, bq, stream)) ||
        (rc = hiprt_memcpy_htod_async(ds, src + bx + bq, bs, stream)) ||
        (rc = hiprt_memcpy_htod_async(dz, src + bx + bq + bs, bz, stream)))
        return die("hiprt_memcpy_htod_async", rc);
    const hiprt_arg args[21] = {
        ptr_arg(dx), ptr_arg(dq), ptr_arg(ds), ptr_arg(dz), ptr_arg(dy),
        i32_arg(M), i32_arg(N), i32_arg(K), i32_arg(G),
        i32_arg(K), i32_arg(1),          /* stride_am, stride_ak */
        i32_arg(N / 8), i32_arg(1),      /* stride_qwk, stride_qwn */
        i32_arg(N), i32_arg(1),          /* stride_sk, stride_sn */
        i32_arg(N / 8), i32_arg(1),      /* stride_qzk, stride_qzn */
        i32_arg(N), i32_arg(1),          /* stride_cm, stride_cn */
        ptr_arg(scratch), ptr_arg(scratch)};
    const uint32_t grid[3] = {(uint32_t)((M + 63) / 64), (uint32_t)((N + 63) / 64), 1};
    const uint32_t block[3] = {256, 1, 1};
    if ((rc = hiprt_launch(ctx, mod, "awq_gemm_int4_typed", grid, block, 0, stream, args, 21)))
        return die("hiprt_launch", rc);
    /* a name the module lacks is reported, not launched */
    if (hiprt_launch(ctx, mod, "no_such_kernel", grid, block, 0, stream, args, 21) != W4A16_ERR_NOT_FOUND) {
        fprintf(stderr, "missing kernel not reported\n");
        return 1;
    }
    if ((rc = hiprt_stream_synchronize(stream))) return die("hiprt_stream_synchronize", rc);
    void* y = malloc(by);
    if ((rc = hiprt_memcpy_dtoh_async(y, dy, by, stream))) return die("hiprt_memcpy_dtoh_async", rc);
    if ((rc = hiprt_stream_synchronize(stream))) return die("hiprt_stream_synchronize", rc);
    FILE* f = fopen(argv[3], "wb");
    if (!f || fwrite(y, 1, by, f) != by) { fprintf(stderr, "cannot write output\n"); return 2; }
    fclose(f);
    const uint64_t bufs[6] = {dx, dq, ds, dz, dy, scratch};
    for (int i = 0; i < 6; ++i)
        if ((rc = hiprt_free(ctx, bufs[i]))) return die("hiprt_free", rc);
    if ((rc = hiprt_stream_destroy(stream))) return die("hiprt_stream_destroy", rc);
    if ((rc = hiprt_module_unload(mod))) return die("hiprt_module_unload", rc);
    if ((rc = hiprt_destroy(ctx))) return die("hiprt_destroy", rc);
    free(in);
    free(y);
    printf("replay_hiprt: M=%d N=%d K=%d G=%d launched and read back\n", M, N, K, G);
    return 0;
}
