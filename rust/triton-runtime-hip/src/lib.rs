//! HIP backend of triton-rs's `DeviceRuntime` (crates/triton-runtime/src/lib.rs:64-85) for
//! AMD Instinct MI355X (gfx950), over libw4a16's C ABI (`include/w4a16.h`), plus safe
//! wrappers of the W4A16 op-level entry points a GPTQ/AWQ linear layer calls.
//!
//! * `HipRuntime::load_module` / `launch` forward to `hiprt_module_load` / `hiprt_launch`;
//!   `KernelArg` values become `hiprt_arg` tagged-union entries in the same order, so a caller
//!   that launches the reference's Triton kernels by name keeps its argument lists and swaps
//!   the binary for `w4a16_typed.hsaco` (kernels `w4a16_gptq_gemm_typed` and
//!   `awq_gemm_int4_typed` with the reference's 19 parameters and Triton's two trailing
//!   scratch pointers).
//! * Status codes map one-to-one onto `RuntimeError` variants; nothing panics across the FFI.
//! * The context is shareable between threads; a stream is used by one thread at a time.

use std::ffi::{c_char, c_void, CStr, CString};

use triton_runtime::{Block, DeviceRuntime, Grid, KernelArg, RuntimeError};

/// `hiprt_arg` (include/w4a16.h): KernelArg as a tagged union.
#[repr(C)]
#[derive(Clone, Copy)]
union HiprtValue {
    i32_: i32,
    u32_: u32,
    i64_: i64,
    f32_: f32,
    device_ptr: u64,
    bytes: *const c_void,
}

#[repr(C)]
#[derive(Clone, Copy)]
struct HiprtArg {
    kind: i32,
    size: u32,
    v: HiprtValue,
}

const ARG_I32: i32 = 0;
const ARG_U32: i32 = 1;
const ARG_I64: i32 = 2;
const ARG_F32: i32 = 3;
const ARG_DEVICE_PTR: i32 = 4;
const ARG_BYTES: i32 = 5;

/// Weight packings (`w4a16_format`).
#[repr(i32)]
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Format {
    /// qweight i32 [K/8, N], zero = nibble + gptq_zero_offset.
    Gptq = 0,
    /// GPTQ with zero 8 and no qzeros.
    GptqSym = 1,
    /// qweight i32 [K, N/8], nibble order [0,4,1,5,2,6,3,7], zero = nibble.
    Awq = 2,
}

#[link(name = "w4a16")]
extern "C" {
    fn w4a16_last_error() -> *const c_char;
    fn w4a16_init(device: i32) -> i32;
    fn hiprt_create(device: i32, out: *mut *mut c_void) -> i32;
    fn hiprt_destroy(ctx: *mut c_void) -> i32;
    fn hiprt_module_load(ctx: *mut c_void, binary: *const c_void, size: usize,
                         out: *mut *mut c_void) -> i32;
    fn hiprt_module_unload(module: *mut c_void) -> i32;
    fn hiprt_launch(ctx: *mut c_void, module: *const c_void, name: *const c_char,
                    grid: *const u32, block: *const u32, shmem: u32, stream: *mut c_void,
                    args: *const HiprtArg, nargs: usize) -> i32;
    fn hiprt_stream_create(ctx: *mut c_void, stream: *mut *mut c_void) -> i32;
    fn hiprt_stream_destroy(stream: *mut c_void) -> i32;
    fn hiprt_stream_synchronize(stream: *mut c_void) -> i32;
    fn hiprt_malloc(ctx: *mut c_void, bytes: usize, ptr: *mut u64) -> i32;
    fn hiprt_free(ctx: *mut c_void, ptr: u64) -> i32;
    fn hiprt_memcpy_htod_async(dst: u64, src: *const c_void, bytes: usize,
                               stream: *mut c_void) -> i32;
    fn hiprt_memcpy_dtoh_async(dst: *mut c_void, src: u64, bytes: usize,
                               stream: *mut c_void) -> i32;
    fn w4a16_gemm(stream: *mut c_void, fmt: i32, x: u64, qweight: u64, scales: u64, qzeros: u64,
                  g_idx: u64, out: u64, m: i32, n: i32, k: i32, group_size: i32,
                  gptq_zero_offset: i32) -> i32;
    fn w4a16_gemm_noalloc(stream: *mut c_void, fmt: i32, x: u64, qweight: u64, scales: u64,
                          qzeros: u64, g_idx: u64, out: u64, m: i32, n: i32, k: i32,
                          group_size: i32, gptq_zero_offset: i32) -> i32;
    fn w4a16_prepare_act_order(stream: *mut c_void, fmt: i32, qweight: u64, g_idx: u64, k: i32,
                               n: i32, group_size: i32, qweight_out: u64, perm_out: u64) -> i32;
    fn w4a16_gemm_act_order(stream: *mut c_void, fmt: i32, x: u64, qweight: u64, scales: u64,
                            qzeros: u64, perm: u64, out: u64, m: i32, n: i32, k: i32,
                            group_size: i32, gptq_zero_offset: i32) -> i32;
    fn w4a16_prepared_bytes(k: i32, n: i32, group_size: i32) -> usize;
    fn w4a16_prepare_layout(stream: *mut c_void, fmt: i32, qweight: u64, scales: u64, qzeros: u64,
                            k: i32, n: i32, group_size: i32, gptq_zero_offset: i32,
                            prepared: u64, prepared_bytes: usize) -> i32;
    fn w4a16_gemm_prepared(stream: *mut c_void, x: u64, prepared: u64, perm: u64, out: u64,
                           m: i32, n: i32, k: i32, group_size: i32) -> i32;
    fn w4a16_dequant_prepared(stream: *mut c_void, prepared: u64, out: u64, k: i32, n: i32,
                              group_size: i32, transposed: i32) -> i32;
    fn w4a16_fused_moe_workspace_size(t: i32, e: i32, topk: i32, i: i32, k: i32,
                                      block_m: i32) -> usize;
    fn w4a16_fused_moe(stream: *mut c_void, fmt: i32, x: u64, router_logits: u64, t: i32, k: i32,
                       i: i32, e: i32, topk: i32, renormalize: i32, w13_qweight: u64,
                       w13_scales: u64, w13_qzeros: u64, w2_qweight: u64, w2_scales: u64,
                       w2_qzeros: u64, group_size: i32, block_m: i32, gptq_zero_offset: i32,
                       workspace: u64, workspace_bytes: usize, out: u64) -> i32;
    fn fused_silu_mul_interleaved_f16(stream: *mut c_void, gate_up: u64, out: u64, inter: i32,
                                      total: i32) -> i32;
    fn fused_silu_mul_interleaved_f32(stream: *mut c_void, gate_up: u64, out: u64, inter: i32,
                                      total: i32) -> i32;
}

/// The calling thread's last libw4a16 message, mapped onto the reference's error type:
/// 1, 2, 5 -> InvalidLaunchConfig; 4, 7 -> ModuleLoad; 6 -> BackendDisabled; else Device.
fn err(code: i32) -> RuntimeError {
    // SAFETY: w4a16_last_error returns a NUL-terminated thread-local string.
    let msg = unsafe { CStr::from_ptr(w4a16_last_error()) }.to_string_lossy().into_owned();
    match code {
        4 | 7 => RuntimeError::ModuleLoad(msg),
        1 | 2 | 5 => RuntimeError::InvalidLaunchConfig(msg),
        6 => RuntimeError::BackendDisabled("hip"),
        _ => RuntimeError::Device(msg),
    }
}

fn check(code: i32) -> Result<(), RuntimeError> {
    if code == 0 { Ok(()) } else { Err(err(code)) }
}

/// A libw4a16 runtime context bound to one device.
pub struct HipRuntime {
    ctx: *mut c_void,
}

/// A loaded gfx950 code object; unloaded on drop.
pub struct HipModule(*mut c_void);

/// A HIP stream (`hipStream_t`); null is the default stream.
pub struct HipStream(pub *mut c_void);

// SAFETY: the library's context is internally synchronised and shareable; modules are
// immutable once loaded; a stream handle is only an identifier (ordering is the caller's).
unsafe impl Send for HipRuntime {}
unsafe impl Sync for HipRuntime {}
unsafe impl Send for HipModule {}
unsafe impl Sync for HipModule {}
unsafe impl Send for HipStream {}
unsafe impl Sync for HipStream {}

impl HipRuntime {
    /// Bind to `device` and run the library's one-time set-up (placement probe, the
    /// allocation-free entry point's scratch), so later calls may be graph-captured.
    pub fn new(device: i32) -> Result<Self, RuntimeError> {
        let mut ctx = std::ptr::null_mut();
        // SAFETY: out-pointer to a local.
        check(unsafe { hiprt_create(device, &mut ctx) })?;
        let rt = Self { ctx };
        // SAFETY: plain call; the device exists (hiprt_create succeeded).
        check(unsafe { w4a16_init(device) })?;
        Ok(rt)
    }

    /// A new stream on this context's device.
    pub fn create_stream(&self) -> Result<HipStream, RuntimeError> {
        let mut s = std::ptr::null_mut();
        // SAFETY: out-pointer to a local.
        check(unsafe { hiprt_stream_create(self.ctx, &mut s) })?;
        Ok(HipStream(s))
    }

    /// Destroy a stream made by `create_stream`.
    pub fn destroy_stream(&self, stream: HipStream) -> Result<(), RuntimeError> {
        // SAFETY: the handle came from hiprt_stream_create and is consumed.
        check(unsafe { hiprt_stream_destroy(stream.0) })
    }

    /// Wait for all work queued on `stream`.
    pub fn synchronize(&self, stream: &HipStream) -> Result<(), RuntimeError> {
        // SAFETY: valid (or null) stream handle.
        check(unsafe { hiprt_stream_synchronize(stream.0) })
    }

    /// Device allocation of `bytes`; the device address.
    pub fn malloc(&self, bytes: usize) -> Result<u64, RuntimeError> {
        let mut p = 0u64;
        // SAFETY: out-pointer to a local.
        check(unsafe { hiprt_malloc(self.ctx, bytes, &mut p) })?;
        Ok(p)
    }

    /// Free an allocation made by `malloc`.
    pub fn free(&self, ptr: u64) -> Result<(), RuntimeError> {
        // SAFETY: the library validates the context; ptr came from hiprt_malloc.
        check(unsafe { hiprt_free(self.ctx, ptr) })
    }

    /// Host -> device copy, asynchronous on `stream`; `src` must stay alive until the stream
    /// has been synchronised.
    pub fn copy_htod(&self, dst: u64, src: &[u8], stream: &HipStream) -> Result<(), RuntimeError> {
        // SAFETY: src is a live slice of src.len() bytes.
        check(unsafe { hiprt_memcpy_htod_async(dst, src.as_ptr().cast(), src.len(), stream.0) })
    }

    /// Device -> host copy, asynchronous on `stream`.
    pub fn copy_dtoh(&self, dst: &mut [u8], src: u64, stream: &HipStream) -> Result<(), RuntimeError> {
        // SAFETY: dst is a live, writable slice of dst.len() bytes.
        check(unsafe { hiprt_memcpy_dtoh_async(dst.as_mut_ptr().cast(), src, dst.len(), stream.0) })
    }
}

impl Drop for HipRuntime {
    fn drop(&mut self) {
        // SAFETY: ctx came from hiprt_create and is destroyed once.
        unsafe { hiprt_destroy(self.ctx) };
    }
}

impl Drop for HipModule {
    fn drop(&mut self) {
        // SAFETY: the handle came from hiprt_module_load and is unloaded once.
        unsafe { hiprt_module_unload(self.0) };
    }
}

fn pack(args: &[KernelArg<'_>]) -> Result<Vec<HiprtArg>, RuntimeError> {
    args.iter()
        .map(|a| {
            Ok(match *a {
                KernelArg::I32(v) => HiprtArg { kind: ARG_I32, size: 0, v: HiprtValue { i32_: v } },
                KernelArg::U32(v) => HiprtArg { kind: ARG_U32, size: 0, v: HiprtValue { u32_: v } },
                KernelArg::I64(v) => HiprtArg { kind: ARG_I64, size: 0, v: HiprtValue { i64_: v } },
                KernelArg::F32(v) => HiprtArg { kind: ARG_F32, size: 0, v: HiprtValue { f32_: v } },
                KernelArg::DevicePtr(p) => {
                    HiprtArg { kind: ARG_DEVICE_PTR, size: 0, v: HiprtValue { device_ptr: p } }
                }
                KernelArg::Bytes(b) => {
                    let size = u32::try_from(b.len()).map_err(|_| {
                        RuntimeError::InvalidLaunchConfig("byte argument above 4 GiB".into())
                    })?;
                    HiprtArg { kind: ARG_BYTES, size, v: HiprtValue { bytes: b.as_ptr().cast() } }
                }
            })
        })
        .collect()
}

impl DeviceRuntime for HipRuntime {
    type Module = HipModule;
    type Stream = HipStream;

    fn load_module(&self, binary: &[u8]) -> Result<HipModule, RuntimeError> {
        let mut m = std::ptr::null_mut();
        // SAFETY: binary is borrowed for the call; the library copies what it keeps.
        check(unsafe { hiprt_module_load(self.ctx, binary.as_ptr().cast(), binary.len(), &mut m) })?;
        Ok(HipModule(m))
    }

    fn launch(&self, module: &HipModule, kernel_name: &str, grid: Grid, block: Block,
              shared_mem_bytes: u32, stream: &HipStream, args: &[KernelArg<'_>])
              -> Result<(), RuntimeError> {
        let packed = pack(args)?;
        let name = CString::new(kernel_name)
            .map_err(|_| RuntimeError::InvalidLaunchConfig("kernel name has a NUL byte".into()))?;
        // SAFETY: every pointer is live for the call; the library copies the argument bytes
        // into the kernel parameter buffer before returning.
        check(unsafe {
            hiprt_launch(self.ctx, module.0, name.as_ptr(), grid.as_ptr(), block.as_ptr(),
                         shared_mem_bytes, stream.0, packed.as_ptr(), packed.len())
        })
    }
}

/// Device addresses of one int4 weight matrix in a checkpoint layout.
#[derive(Debug, Clone, Copy)]
pub struct QuantWeights {
    /// Packed nibbles (GPTQ [K/8, N] or AWQ [K, N/8] i32).
    pub qweight: u64,
    /// fp16 [K/G, N].
    pub scales: u64,
    /// i32 [K/G, N/8], or 0 for `Format::GptqSym`.
    pub qzeros: u64,
}

/// out[M, N] = x[M, K] @ W16 on `stream` (fp32 accumulate, fp16 out); `g_idx` 0 when absent.
/// The kernel is chosen by shape (decode GEMV, small-batch MFMA, prefill MFMA).
#[allow(clippy::too_many_arguments)]
pub fn gemm(stream: &HipStream, fmt: Format, x: u64, w: &QuantWeights, g_idx: u64, out: u64,
            m: i32, n: i32, k: i32, group_size: i32, gptq_zero_offset: i32)
            -> Result<(), RuntimeError> {
    // SAFETY: device addresses are opaque to the host; the library validates sizes first.
    check(unsafe {
        w4a16_gemm(stream.0, fmt as i32, x, w.qweight, w.scales, w.qzeros, g_idx, out, m, n, k,
                   group_size, gptq_zero_offset)
    })
}

/// As `gemm`, allocating nothing (for code under graph capture): the split-K scratch is a
/// fixed per-device array; calls that overlap on one device must be serialised.
#[allow(clippy::too_many_arguments)]
pub fn gemm_noalloc(stream: &HipStream, fmt: Format, x: u64, w: &QuantWeights, g_idx: u64,
                    out: u64, m: i32, n: i32, k: i32, group_size: i32, gptq_zero_offset: i32)
                    -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe {
        w4a16_gemm_noalloc(stream.0, fmt as i32, x, w.qweight, w.scales, w.qzeros, g_idx, out, m,
                           n, k, group_size, gptq_zero_offset)
    })
}

/// One-time act-order repack: `qweight_out` = rows in group order, `perm_out` = the order.
/// Synchronises `stream`.
#[allow(clippy::too_many_arguments)]
pub fn prepare_act_order(stream: &HipStream, fmt: Format, qweight: u64, g_idx: u64, k: i32,
                         n: i32, group_size: i32, qweight_out: u64, perm_out: u64)
                         -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe {
        w4a16_prepare_act_order(stream.0, fmt as i32, qweight, g_idx, k, n, group_size,
                                qweight_out, perm_out)
    })
}

/// x @ W16 for an act-order checkpoint prepared by `prepare_act_order`.
#[allow(clippy::too_many_arguments)]
pub fn gemm_act_order(stream: &HipStream, fmt: Format, x: u64, w_prepared: &QuantWeights,
                      perm: u64, out: u64, m: i32, n: i32, k: i32, group_size: i32,
                      gptq_zero_offset: i32) -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe {
        w4a16_gemm_act_order(stream.0, fmt as i32, x, w_prepared.qweight, w_prepared.scales,
                             w_prepared.qzeros, perm, out, m, n, k, group_size, gptq_zero_offset)
    })
}

/// Bytes of the prepared layout of a K x N matrix (0: shape not supported: N % 16, K % 128,
/// K <= 32768, group size 32, 64 or a multiple of 128).
pub fn prepared_bytes(k: i32, n: i32, group_size: i32) -> usize {
    // SAFETY: pure function of its arguments.
    unsafe { w4a16_prepared_bytes(k, n, group_size) }
}

/// One-time rewrite of a checkpoint matrix into the prepared layout at `prepared` (256-byte
/// aligned, `prepared_bytes` long, not overlapping the checkpoint). Asynchronous on `stream`.
#[allow(clippy::too_many_arguments)]
pub fn prepare_layout(stream: &HipStream, fmt: Format, w: &QuantWeights, k: i32, n: i32,
                      group_size: i32, gptq_zero_offset: i32, prepared: u64,
                      prepared_bytes: usize) -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe {
        w4a16_prepare_layout(stream.0, fmt as i32, w.qweight, w.scales, w.qzeros, k, n,
                             group_size, gptq_zero_offset, prepared, prepared_bytes)
    })
}

/// out[M, N] = x[M, K] @ W16 from prepared weights, any M; `perm` 0, or the permutation of an
/// act-order checkpoint repacked by `prepare_act_order` before `prepare_layout`.
#[allow(clippy::too_many_arguments)]
pub fn gemm_prepared(stream: &HipStream, x: u64, prepared: u64, perm: u64, out: u64, m: i32,
                     n: i32, k: i32, group_size: i32) -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe { w4a16_gemm_prepared(stream.0, x, prepared, perm, out, m, n, k, group_size) })
}

/// The fp16 weights of a prepared matrix, [K, N] or (transposed) [N, K], bit-exact.
pub fn dequant_prepared(stream: &HipStream, prepared: u64, out: u64, k: i32, n: i32,
                        group_size: i32, transposed: bool) -> Result<(), RuntimeError> {
    // SAFETY: as for gemm.
    check(unsafe {
        w4a16_dequant_prepared(stream.0, prepared, out, k, n, group_size, transposed as i32)
    })
}

/// Shape of a fused-MoE layer.
#[derive(Debug, Clone, Copy)]
pub struct MoeShape {
    /// Tokens.
    pub tokens: i32,
    /// Hidden size (x and y columns).
    pub hidden: i32,
    /// Expert FFN width.
    pub inter: i32,
    /// Experts.
    pub experts: i32,
    /// Experts per token.
    pub topk: i32,
    /// Quantisation group size.
    pub group_size: i32,
    /// Routing-table block (64 or 128).
    pub block_m: i32,
}

/// Bytes of device workspace `fused_moe` needs.
pub fn fused_moe_workspace_size(s: &MoeShape) -> usize {
    // SAFETY: pure function of its arguments.
    unsafe { w4a16_fused_moe_workspace_size(s.tokens, s.experts, s.topk, s.inter, s.hidden, s.block_m) }
}

/// Whole MoE layer: route, align, grouped GEMM (w1|w3), silu*mul, grouped GEMM (w2), combine.
#[allow(clippy::too_many_arguments)]
pub fn fused_moe(stream: &HipStream, fmt: Format, s: &MoeShape, x: u64, router_logits: u64,
                 renormalize: bool, w13: &QuantWeights, w2: &QuantWeights, gptq_zero_offset: i32,
                 workspace: u64, workspace_bytes: usize, out: u64) -> Result<(), RuntimeError> {
    // SAFETY: as for gemm; the workspace size is checked by the library.
    check(unsafe {
        w4a16_fused_moe(stream.0, fmt as i32, x, router_logits, s.tokens, s.hidden, s.inter,
                        s.experts, s.topk, renormalize as i32, w13.qweight, w13.scales,
                        w13.qzeros, w2.qweight, w2.scales, w2.qzeros, s.group_size, s.block_m,
                        gptq_zero_offset, workspace, workspace_bytes, out)
    })
}

/// `fused_silu_mul_interleaved_f16` (elementwise.rs:188-212): `out[b*inter+i] =
/// f16(silu(g) * u)`, `g = gate_up[b*2*inter+i]`, `u = gate_up[b*2*inter+inter+i]`.
pub fn silu_mul_interleaved_f16(stream: &HipStream, gate_up: u64, out: u64, inter: i32,
                                total: i32) -> Result<(), RuntimeError> {
    // SAFETY: device pointers from hiprt_malloc; the library validates the sizes.
    check(unsafe { fused_silu_mul_interleaved_f16(stream.0, gate_up, out, inter, total) })
}

/// `fused_silu_mul_interleaved_f32` (elementwise.rs:214-250): the same over f32 buffers.
pub fn silu_mul_interleaved_f32(stream: &HipStream, gate_up: u64, out: u64, inter: i32,
                                total: i32) -> Result<(), RuntimeError> {
    // SAFETY: as above.
    check(unsafe { fused_silu_mul_interleaved_f32(stream.0, gate_up, out, inter, total) })
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn packs_kernel_args_in_order() {
        let bytes = [1u8, 2, 3];
        let p = pack(&[KernelArg::I32(-3), KernelArg::U32(7), KernelArg::I64(1 << 40),
                       KernelArg::F32(0.5), KernelArg::DevicePtr(0xdead_beef),
                       KernelArg::Bytes(&bytes)]).unwrap();
        assert_eq!(p.iter().map(|a| a.kind).collect::<Vec<_>>(), vec![0, 1, 2, 3, 4, 5]);
        // SAFETY: reading the union member written for each kind.
        unsafe {
            assert_eq!(p[0].v.i32_, -3);
            assert_eq!(p[2].v.i64_, 1 << 40);
            assert_eq!(p[4].v.device_ptr, 0xdead_beef);
        }
        assert_eq!(p[5].size, 3);
    }

    /// Needs an MI355X and a built libw4a16 (W4A16_LIB_DIR): `cargo test -- --ignored`.
    #[test]
    #[ignore]
    fn bad_module_is_a_module_load_error() {
        let rt = HipRuntime::new(0).unwrap();
        assert!(matches!(rt.load_module(b"not a code object"), Err(RuntimeError::ModuleLoad(_))));
    }
}
