"""Python host side of the MI355X W4A16 library (ctypes over libw4a16.so, include/w4a16.h).

Mirrors the reference's launch interface for this path: the kernel-level functions keep
the parameter lists of `w4a16_gptq_gemm_typed` and `awq_gemm_int4_typed`
(crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:103-129,
awq_gemm_int4_typed.rs:94-115) and of the two dequant kernels
(ferrum_dequant_int4.rs:27-37, ferrum_dequant_int4_sym.rs:24-31); `HipRuntime` mirrors the
DeviceRuntime trait (crates/triton-runtime/src/lib.rs:64-85) with RuntimeError-style
exceptions. Tensors are torch tensors on the GPU (torch provides memory and streams);
every computation runs in the HIP library, and loading fails loudly when it is missing.
"""
from __future__ import annotations

import ctypes
import os

import torch  # loaded first so the process has one HIP runtime (same SONAME)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libw4a16.so")
HSACO_PATH = os.path.join(HERE, "w4a16_typed.hsaco")
META_PATH = os.path.join(HERE, "w4a16_typed.json")

FMT_GPTQ, FMT_GPTQ_SYM, FMT_AWQ = 0, 1, 2
BF16 = 0x100   # W4A16_BF16: bfloat16 activations, scales and output (OR-ed into the format)
FORMATS = {"gptq": FMT_GPTQ, "gptq_sym": FMT_GPTQ_SYM, "awq": FMT_AWQ}
KERNELS = {1: "gemv", 2: "skinny", 3: "prefill", 4: "strided"}

OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_DEVICE, ERR_MODULE_LOAD, ERR_LAUNCH_CONFIG, \
    ERR_BACKEND_DISABLED, ERR_NOT_FOUND = range(8)


class RuntimeError_(RuntimeError):
    """Base of the runtime errors (crates/triton-runtime/src/lib.rs:18-35)."""

    code = -1


class InvalidArgument(RuntimeError_, ValueError):
    code = ERR_INVALID_ARG


class Unsupported(RuntimeError_):
    code = ERR_UNSUPPORTED


class DeviceError(RuntimeError_):
    code = ERR_DEVICE


class ModuleLoad(RuntimeError_):
    code = ERR_MODULE_LOAD


class InvalidLaunchConfig(RuntimeError_):
    code = ERR_LAUNCH_CONFIG


class BackendDisabled(RuntimeError_):
    code = ERR_BACKEND_DISABLED


class NotFound(RuntimeError_):
    code = ERR_NOT_FOUND


_ERRORS = {c.code: c for c in (InvalidArgument, Unsupported, DeviceError, ModuleLoad,
                               InvalidLaunchConfig, BackendDisabled, NotFound)}

EXPORTED = (
    "w4a16_last_error", "w4a16_version", "w4a16_init", "w4a16_gemm", "w4a16_gemm_noalloc",
    "w4a16_gemm_noalloc_scratch_bytes", "w4a16_gemm_plan", "w4a16_prepare_act_order",
    "w4a16_gemm_act_order", "w4a16_prepared_bytes", "w4a16_prepare_layout",
    "w4a16_gemm_prepared", "w4a16_dequant_prepared", "w4a16_gemm_prepared_gidx",
    "w4a16_typed_plan",
    "w4a16_gptq_gemm_typed", "awq_gemm_int4_typed", "dequant_int4_to_fp16",
    "dequant_int4_sym_to_fp16", "w4a16_dequant", "w4a16_moe_route", "w4a16_moe_align",
    "w4a16_moe_gemm", "fused_silu_mul_interleaved_f16", "fused_silu_mul_interleaved_f32",
    "w4a16_moe_sum",
    "w4a16_fused_moe_workspace_size", "w4a16_fused_moe", "w4a16_fused_moe_prepared",
    "hiprt_create", "hiprt_destroy", "hiprt_module_load", "hiprt_module_unload", "hiprt_launch",
    "hiprt_stream_create", "hiprt_stream_destroy", "hiprt_stream_synchronize", "hiprt_malloc",
    "hiprt_free", "hiprt_memcpy_htod_async", "hiprt_memcpy_dtoh_async", "hiprt_memset_async",
    "hiprt_event_create", "hiprt_event_destroy", "hiprt_event_record", "hiprt_event_synchronize",
    "hiprt_event_elapsed_ms",
)

_lib = None
_P, _I, _Z = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t


def lib() -> ctypes.CDLL:
    """Load libw4a16.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python triton-rs_amd/build.py` "
                              "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        L.w4a16_last_error.restype = ctypes.c_char_p
        L.w4a16_version.restype = ctypes.c_char_p
        L.w4a16_gemm.argtypes = [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.w4a16_gemm_plan.argtypes = [_I, _I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_int)]
        L.w4a16_init.argtypes = [_I]
        L.w4a16_prepare_act_order.argtypes = [_P, _I, _P, _P, _I, _I, _I, _P, _P]
        L.w4a16_gemm_act_order.argtypes = [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.w4a16_prepared_bytes.restype = ctypes.c_size_t
        L.w4a16_prepared_bytes.argtypes = [_I, _I, _I]
        L.w4a16_prepare_layout.argtypes = [_P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _Z]
        L.w4a16_gemm_prepared.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I]
        L.w4a16_gemm_prepared_gidx.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I]
        L.w4a16_dequant_prepared.argtypes = [_P, _P, _P, _I, _I, _I, _I]
        L.w4a16_gemm_noalloc.argtypes = [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.w4a16_gemm_noalloc_scratch_bytes.restype = ctypes.c_size_t
        L.w4a16_gemm_noalloc_scratch_bytes.argtypes = []
        L.w4a16_typed_plan.argtypes = [_I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_int32), _I,
                                       ctypes.POINTER(ctypes.c_int)]
        L.w4a16_gptq_gemm_typed.argtypes = [_P] * 6 + [_I] * 14
        L.awq_gemm_int4_typed.argtypes = [_P] * 6 + [_I] * 14
        L.dequant_int4_to_fp16.argtypes = [_P] * 5 + [_I] * 4
        L.dequant_int4_sym_to_fp16.argtypes = [_P] * 4 + [_I] * 3
        L.w4a16_dequant.argtypes = [_P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.w4a16_moe_route.argtypes = [_P, _P, _I, _I, _I, _I, _P, _P]
        L.w4a16_moe_align.argtypes = [_P, _P, _I, _I, _I, _I, _P, _P, _P]
        _L = ctypes.c_int64
        L.w4a16_moe_gemm.argtypes = [_P, _I, _P, _I, _P, _P, _P, _L, _L, _L, _I, _P, _P, _P, _P,
                                     _I, _I, _I, _I, _I, _I, _I]
        L.fused_silu_mul_interleaved_f16.argtypes = [_P, _P, _P, _I, _I]
        L.fused_silu_mul_interleaved_f32.argtypes = [_P, _P, _P, _I, _I]
        L.w4a16_moe_sum.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        L.w4a16_fused_moe_workspace_size.restype = ctypes.c_size_t
        L.w4a16_fused_moe_workspace_size.argtypes = [_I] * 6
        L.w4a16_fused_moe.argtypes = [_P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P,
                                      _P, _I, _I, _I, _P, _Z, _P]
        L.w4a16_fused_moe_prepared.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _I,
                                               _P, _Z, _P]
        L.hiprt_create.argtypes = [_I, ctypes.POINTER(_P)]
        L.hiprt_destroy.argtypes = [_P]
        L.hiprt_module_load.argtypes = [_P, _P, _Z, ctypes.POINTER(_P)]
        L.hiprt_module_unload.argtypes = [_P]
        L.hiprt_launch.argtypes = [_P, _P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                   ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32, _P, _P, _Z]
        L.hiprt_stream_create.argtypes = [_P, ctypes.POINTER(_P)]
        L.hiprt_stream_destroy.argtypes = [_P]
        L.hiprt_stream_synchronize.argtypes = [_P]
        L.hiprt_malloc.argtypes = [_P, _Z, ctypes.POINTER(ctypes.c_uint64)]
        L.hiprt_free.argtypes = [_P, ctypes.c_uint64]
        L.hiprt_memcpy_htod_async.argtypes = [ctypes.c_uint64, _P, _Z, _P]
        L.hiprt_memcpy_dtoh_async.argtypes = [_P, ctypes.c_uint64, _Z, _P]
        L.hiprt_memset_async.argtypes = [ctypes.c_uint64, ctypes.c_int, _Z, _P]
        L.hiprt_event_create.argtypes = [ctypes.POINTER(_P)]
        L.hiprt_event_destroy.argtypes = [_P]
        L.hiprt_event_record.argtypes = [_P, _P]
        L.hiprt_event_synchronize.argtypes = [_P]
        L.hiprt_event_elapsed_ms.argtypes = [_P, _P, ctypes.POINTER(ctypes.c_float)]
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().w4a16_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError_)(msg)


def version() -> str:
    return lib().w4a16_version().decode()


# ------------------------------------------------------------------ tensor plumbing

def _stream(t: torch.Tensor | None = None):
    dev = t.device if t is not None else torch.device("cuda")
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _fmt(fmt) -> int:
    if isinstance(fmt, str):
        return FORMATS[fmt]
    return int(fmt)


def _require(t: torch.Tensor, name: str, dtypes, device: torch.device | None = None):
    if not isinstance(t, torch.Tensor):
        raise InvalidArgument(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise InvalidArgument(f"{name} must be on the GPU")
    if t.dtype not in dtypes:
        raise InvalidArgument(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if device is not None and t.device != device:
        raise InvalidArgument(f"{name} is on {t.device}, expected {device}")


_INT32 = (torch.int32,)
_HALF = (torch.float16,)
_ELEM = (torch.float16, torch.bfloat16)   # element types of x, scales and out


def _gemm_operands(f: int, x, qweight, scales, qzeros, idx, idx_name: str, elem=_HALF):
    """(M, N, K) of a GEMM call after checking dtypes, devices, ranks and contiguity (the C ABI
    takes contiguous row-major buffers and checks sizes, not layouts). x and scales share one
    element type out of `elem`."""
    _require(x, "x", elem)
    dev = x.device
    _require(qweight, "qweight", _INT32, dev)
    _require(scales, "scales", (x.dtype,), dev)
    if qzeros is not None:
        _require(qzeros, "qzeros", _INT32, dev)
    if idx is not None:
        _require(idx, idx_name, _INT32, dev)
    if x.dim() != 2 or qweight.dim() != 2:
        raise InvalidArgument("x and qweight must be 2-D")
    for t, n in ((x, "x"), (qweight, "qweight"), (scales, "scales"), (qzeros, "qzeros"),
                 (idx, idx_name)):
        if t is not None and not t.is_contiguous():
            raise InvalidArgument(f"{n} must be contiguous")
    M, K = x.shape
    N = qweight.shape[1] * 8 if f == FMT_AWQ else qweight.shape[1]
    return M, N, K


def _gemm_out(out, M: int, N: int, dev: torch.device, required: bool = False,
              dtype=torch.float16):
    if out is None:
        if required:
            raise InvalidArgument("out must be given")
        return torch.empty((M, N), dtype=dtype, device=dev)
    _require(out, "out", (dtype,), dev)
    if tuple(out.shape) != (M, N) or not out.is_contiguous():
        raise InvalidArgument(f"out must be a contiguous [{M}, {N}] tensor")
    return out


# ------------------------------------------------------------------ op level

def init(device: int = 0) -> None:
    """Optional per-device set-up (CU count, workgroup-placement probe) ahead of graph capture."""
    check(lib().w4a16_init(device))


def typed_plan(fmt, m: int, n: int, k: int, group_size: int, strides, aligned16: bool = True) -> str:
    """Kernel regime the reference-named typed entry points would run for these strides."""
    k_ = ctypes.c_int(0)
    arr = (ctypes.c_int32 * 10)(*strides)
    check(lib().w4a16_typed_plan(_fmt(fmt), m, n, k, group_size, arr, int(aligned16),
                                 ctypes.byref(k_)))
    return KERNELS[k_.value]


def plan(fmt, M: int, N: int, K: int, group_size: int, has_g_idx: bool = False,
         bf16: bool = False) -> str:
    """Name of the kernel regime w4a16_gemm would choose (no GPU access)."""
    k = ctypes.c_int(0)
    f = _fmt(fmt) | (BF16 if bf16 else 0)
    check(lib().w4a16_gemm_plan(f, M, N, K, group_size, int(has_g_idx), ctypes.byref(k)))
    return KERNELS[k.value]


def _elem_flag(x: torch.Tensor) -> int:
    return BF16 if x.dtype == torch.bfloat16 else 0


def gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
         qzeros: torch.Tensor | None, fmt="awq", group_size: int = 128,
         g_idx: torch.Tensor | None = None, out: torch.Tensor | None = None,
         zero_offset: int = 1) -> torch.Tensor:
    """out[M, N] = x[M, K] @ dequant(qweight) with fp32 accumulation, in fp16 or, when x and
    scales are bfloat16, in bfloat16 (the same kernels as fp16, act-order included).

    fmt: "gptq" (qweight int32 [K/8, N], qzeros [K/G, N/8], zero = nibble + zero_offset),
    "gptq_sym" (zero = 8, qzeros unused) or "awq" (qweight [K, N/8], AWQ nibble order).
    """
    f = _fmt(fmt)
    M, N, K = _gemm_operands(f, x, qweight, scales, qzeros, g_idx, "g_idx", _ELEM)
    out = _gemm_out(out, M, N, x.device, dtype=x.dtype)
    check(lib().w4a16_gemm(_stream(x), f | _elem_flag(x), _ptr(x), _ptr(qweight), _ptr(scales),
                           _ptr(qzeros), _ptr(g_idx), _ptr(out), M, N, K, group_size,
                           zero_offset))
    return out


def prepare_act_order(qweight: torch.Tensor, g_idx: torch.Tensor, group_size: int = 128,
                      fmt="gptq"):
    """(qweight in group order, perm): the one-time act-order repack (synchronises)."""
    f = _fmt(fmt)
    _require(qweight, "qweight", _INT32)
    _require(g_idx, "g_idx", _INT32, qweight.device)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    qout = torch.empty_like(qweight)
    perm = torch.empty(K, dtype=torch.int32, device=qweight.device)
    check(lib().w4a16_prepare_act_order(_stream(qweight), f, _ptr(qweight.contiguous()),
                                        _ptr(g_idx.contiguous()), K, N, group_size, _ptr(qout),
                                        _ptr(perm)))
    return qout, perm


def gemm_act_order(x, qweight_prepared, scales, qzeros, perm, fmt="gptq", group_size: int = 128,
                   zero_offset: int = 1, out=None) -> torch.Tensor:
    """x @ W16 for an act-order checkpoint prepared by prepare_act_order."""
    f = _fmt(fmt)
    M, N, K = _gemm_operands(f, x, qweight_prepared, scales, qzeros, perm, "perm")
    out = _gemm_out(out, M, N, x.device)
    check(lib().w4a16_gemm_act_order(_stream(x), f, _ptr(x), _ptr(qweight_prepared), _ptr(scales),
                                     _ptr(qzeros), _ptr(perm), _ptr(out), M, N, K, group_size,
                                     zero_offset))
    return out


class PreparedWeights:
    """A weight matrix in the prepared layout (w4a16_prepare_layout): a uint8 device buffer
    plus the (K, N, group_size) it was made for. The checkpoint's format and zero convention
    are folded into it."""

    def __init__(self, buffer: torch.Tensor, K: int, N: int, group_size: int):
        self.buffer, self.K, self.N, self.group_size = buffer, K, N, group_size


def prepared_bytes(K: int, N: int, group_size: int = 128) -> int:
    """Bytes of the prepared layout for this shape (0: shape not supported)."""
    return lib().w4a16_prepared_bytes(K, N, group_size)


def prepare_layout(qweight, scales, qzeros, fmt="awq", group_size: int = 128,
                   zero_offset: int = 1) -> PreparedWeights:
    """One-time rewrite of a GPTQ / GPTQ_SYM / AWQ checkpoint into the prepared layout."""
    f = _fmt(fmt)
    _require(qweight, "qweight", _INT32)
    dev = qweight.device
    _require(scales, "scales", _HALF, dev)
    if qzeros is not None:
        _require(qzeros, "qzeros", _INT32, dev)
    for t, n in ((qweight, "qweight"), (scales, "scales"), (qzeros, "qzeros")):
        if t is not None and not t.is_contiguous():
            raise InvalidArgument(f"{n} must be contiguous")
    if f == FMT_AWQ:
        K, N = qweight.shape[0], qweight.shape[1] * 8
    else:
        K, N = qweight.shape[0] * 8, qweight.shape[1]
    nbytes = prepared_bytes(K, N, group_size)
    if nbytes == 0:
        raise Unsupported(f"no prepared layout for K={K} N={N} group_size={group_size}")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    check(lib().w4a16_prepare_layout(_stream(qweight), f, _ptr(qweight), _ptr(scales),
                                     _ptr(qzeros), K, N, group_size, zero_offset, _ptr(buf),
                                     nbytes))
    return PreparedWeights(buf, K, N, group_size)


def gemm_prepared(x: torch.Tensor, w: PreparedWeights, perm: torch.Tensor | None = None,
                  out: torch.Tensor | None = None, g_idx: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = x[M, K] @ W16 from prepared weights (perm: an act-order checkpoint repacked
    by prepare_act_order before prepare_layout; x's columns are gathered by it first. g_idx:
    an act-order checkpoint prepared as stored, g_idx[k] the group of row k
    (w4a16_gemm_prepared_gidx))."""
    if perm is not None and g_idx is not None:
        raise InvalidArgument("give perm (group-order repack) or g_idx (rows as stored), not both")
    _require(x, "x", _HALF)
    if perm is not None:
        _require(perm, "perm", _INT32, x.device)
    if g_idx is not None:
        _require(g_idx, "g_idx", _INT32, x.device)
        if g_idx.dim() != 1 or g_idx.numel() != w.K or not g_idx.is_contiguous():
            raise InvalidArgument(f"g_idx must be a contiguous int32 vector of K={w.K} entries")
    if x.dim() != 2 or not x.is_contiguous():
        raise InvalidArgument("x must be a contiguous 2-D tensor")
    M, K = x.shape
    if K != w.K:
        raise InvalidArgument(f"x has K={K}, the prepared weights K={w.K}")
    out = _gemm_out(out, M, w.N, x.device)
    if g_idx is not None:
        check(lib().w4a16_gemm_prepared_gidx(_stream(x), _ptr(x), _ptr(w.buffer), _ptr(g_idx),
                                             _ptr(out), M, w.N, K, w.group_size))
        return out
    check(lib().w4a16_gemm_prepared(_stream(x), _ptr(x), _ptr(w.buffer), _ptr(perm), _ptr(out),
                                    M, w.N, K, w.group_size))
    return out


def dequant_prepared(w: PreparedWeights, transposed: bool = False) -> torch.Tensor:
    """fp16 weights of a prepared matrix, [K, N] (or [N, K] when transposed)."""
    out = torch.empty((w.N, w.K) if transposed else (w.K, w.N), dtype=torch.float16,
                      device=w.buffer.device)
    check(lib().w4a16_dequant_prepared(_stream(w.buffer), _ptr(w.buffer), _ptr(out), w.K, w.N,
                                       w.group_size, int(transposed)))
    return out


def gemm_noalloc(x, qweight, scales, qzeros, out, fmt="awq", group_size: int = 128, g_idx=None,
                 zero_offset: int = 1) -> torch.Tensor:
    """w4a16_gemm_noalloc: as gemm(), but the library allocates nothing during the call (its
    split-K scratch is a fixed per-device array); `out` must be given."""
    f = _fmt(fmt)
    M, N, K = _gemm_operands(f, x, qweight, scales, qzeros, g_idx, "g_idx", _ELEM)
    out = _gemm_out(out, M, N, x.device, required=True, dtype=x.dtype)
    check(lib().w4a16_gemm_noalloc(_stream(x), f | _elem_flag(x), _ptr(x), _ptr(qweight),
                                   _ptr(scales), _ptr(qzeros), _ptr(g_idx), _ptr(out), M, N, K,
                                   group_size, zero_offset))
    return out


def dequant(qweight, scales, qzeros, fmt="gptq", K: int | None = None, group_size: int = 128,
            g_idx=None, zero_offset: int = 1, transposed: bool = False) -> torch.Tensor:
    """The dequantised weights, [K, N] (or [N, K] when transposed), in the scales' element
    type (fp16, or bfloat16: RNE_bf16((q - z) * s))."""
    f = _fmt(fmt)
    _require(qweight, "qweight", _INT32)
    dev = qweight.device
    _require(scales, "scales", _ELEM, dev)
    if qzeros is not None:
        _require(qzeros, "qzeros", _INT32, dev)
    if g_idx is not None:
        _require(g_idx, "g_idx", _INT32, dev)
    for t, n in ((qweight, "qweight"), (scales, "scales"), (qzeros, "qzeros"), (g_idx, "g_idx")):
        if t is not None and not t.is_contiguous():
            raise InvalidArgument(f"{n} must be contiguous")
    if f == FMT_AWQ:
        K, N = qweight.shape[0], qweight.shape[1] * 8
    else:
        K, N = qweight.shape[0] * 8, qweight.shape[1]
    out = torch.empty((N, K) if transposed else (K, N), dtype=scales.dtype, device=qweight.device)
    check(lib().w4a16_dequant(_stream(qweight), f | _elem_flag(scales), _ptr(qweight),
                              _ptr(scales), _ptr(qzeros), _ptr(g_idx), _ptr(out), K, N,
                              group_size, zero_offset, int(transposed)))
    return out


# ------------------------------------------------------------------ fused MoE

def moe_route(logits: torch.Tensor, topk: int, renormalize: bool = True):
    """(topk_ids int32 [T, topk], topk_weights fp32 [T, topk]) from fp32 logits [T, E]."""
    _require(logits, "logits", (torch.float32,))
    T, E = logits.shape
    ids = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device)
    check(lib().w4a16_moe_route(_stream(logits), _ptr(logits.contiguous()), T, E, topk,
                                int(renormalize), _ptr(ids), _ptr(w)))
    return ids, w


def moe_capacity(num_pairs: int, E: int, block_m: int) -> int:
    cap = num_pairs + E * (block_m - 1)
    return (cap + block_m - 1) // block_m * block_m


def moe_align(topk_ids: torch.Tensor, E: int, block_m: int = 64):
    """(sorted_ids [capacity], expert_ids [capacity / block_m], num_post_padded [1])."""
    _require(topk_ids, "topk_ids", _INT32)
    P = topk_ids.numel()
    cap = moe_capacity(P, E, block_m)
    dev = topk_ids.device
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(cap // block_m, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib().w4a16_moe_align(_stream(topk_ids), _ptr(topk_ids.contiguous()), P, E, block_m,
                                cap, _ptr(sorted_ids), _ptr(expert_ids), _ptr(npp)))
    return sorted_ids, expert_ids, npp


def moe_gemm(a, a_div, qweight, scales, qzeros, sorted_ids, expert_ids, npp, num_pairs, N, K,
             fmt="gptq", group_size=128, block_m=64, zero_offset=1, out=None):
    """Grouped GEMM: out[p] = a[p // a_div] @ W16[expert of p]; weights stacked [E, ...]."""
    f = _fmt(fmt)
    if out is None:
        out = torch.empty((num_pairs, N), dtype=torch.float16, device=a.device)
    qs = qweight[0].numel()
    ss = scales[0].numel()
    zs = 0 if qzeros is None else qzeros[0].numel()
    check(lib().w4a16_moe_gemm(_stream(a), f, _ptr(a), a_div, _ptr(qweight), _ptr(scales),
                               _ptr(qzeros), qs, ss, zs, qweight.shape[0], _ptr(sorted_ids),
                               _ptr(expert_ids),
                               _ptr(npp), _ptr(out), num_pairs, N, K, group_size, block_m,
                               sorted_ids.numel(), zero_offset))
    return out


def fused_silu_mul_interleaved_f16(gate_up, out, inter, total, stream=None):
    """elementwise.rs:188-212 parameter list: out[b*inter+i] = silu(g)*u."""
    st = stream if stream is not None else _stream(gate_up)
    check(lib().fused_silu_mul_interleaved_f16(st, _p(gate_up), _p(out), inter, total))


def fused_silu_mul_interleaved_f32(gate_up, out, inter, total, stream=None):
    """elementwise.rs:214-250 parameter list over float32 tensors: out[b*inter+i] = silu(g)*u."""
    st = stream if stream is not None else _stream(gate_up)
    check(lib().fused_silu_mul_interleaved_f32(st, _p(gate_up), _p(out), inter, total))


def moe_sum(y_pairs, topk_weights, T, topk, K, out=None):
    if out is None:
        out = torch.empty((T, K), dtype=torch.float16, device=y_pairs.device)
    check(lib().w4a16_moe_sum(_stream(y_pairs), _ptr(y_pairs), _ptr(topk_weights), _ptr(out), T,
                              topk, K))
    return out


def fused_moe(x, router_logits, w13, w2, topk=2, fmt="gptq", group_size=128, block_m=64,
              renormalize=True, zero_offset=1, out=None, workspace=None):
    """Whole MoE layer through w4a16_fused_moe. w13 / w2 are (qweight, scales, qzeros) stacked
    over experts; w13 columns [0, I) are w1 (gate) and [I, 2I) w3 (up)."""
    f = _fmt(fmt)
    T, K = x.shape
    E = router_logits.shape[1]
    q13, s13, z13 = w13
    q2, s2, z2 = w2
    I = s2.shape[1] * group_size
    need = lib().w4a16_fused_moe_workspace_size(T, E, topk, I, K, block_m)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty((T, K), dtype=torch.float16, device=x.device)
    check(lib().w4a16_fused_moe(_stream(x), f, _ptr(x), _ptr(router_logits.contiguous()), T, K, I,
                                E, topk, int(renormalize), _ptr(q13), _ptr(s13), _ptr(z13),
                                _ptr(q2), _ptr(s2), _ptr(z2), group_size, block_m, zero_offset,
                                _ptr(workspace), workspace.numel(), _ptr(out)))
    return out


def prepare_layout_experts(qweight, scales, qzeros, fmt="gptq", group_size: int = 128,
                           zero_offset: int = 1) -> PreparedWeights:
    """Stacked experts ([E] x checkpoint tensors) into one buffer of E consecutive prepared
    matrices (w4a16_prepare_layout per expert), as w4a16_fused_moe_prepared takes them."""
    E = qweight.shape[0]
    f = _fmt(fmt)
    if f == FMT_AWQ:
        K, N = qweight.shape[1], qweight.shape[2] * 8
    else:
        K, N = qweight.shape[1] * 8, qweight.shape[2]
    per = prepared_bytes(K, N, group_size)
    if per == 0:
        raise Unsupported(f"no prepared layout for K={K} N={N} group_size={group_size}")
    buf = torch.empty(E * per, dtype=torch.uint8, device=qweight.device)
    for e in range(E):
        check(lib().w4a16_prepare_layout(_stream(qweight), f, _ptr(qweight[e]), _ptr(scales[e]),
                                         None if qzeros is None else _ptr(qzeros[e]), K, N,
                                         group_size, zero_offset, _ptr(buf[e * per:]), per))
    return PreparedWeights(buf, K, N, group_size)


def fused_moe_prepared(x, router_logits, w13: PreparedWeights, w2: PreparedWeights, topk=2,
                       block_m=64, renormalize=True, out=None, workspace=None):
    """Whole MoE layer through w4a16_fused_moe_prepared: w13 / w2 from prepare_layout_experts
    (K -> 2I and I -> K per expert)."""
    _require(x, "x", _HALF)
    T, K = x.shape
    E = router_logits.shape[1]
    I = w2.K
    if w13.K != K or w13.N != 2 * I or w2.N != K or w13.group_size != w2.group_size:
        raise InvalidArgument("w13 must be K -> 2I and w2 I -> K with one group size")
    G = w13.group_size
    need = lib().w4a16_fused_moe_workspace_size(T, E, topk, I, K, block_m)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty((T, K), dtype=torch.float16, device=x.device)
    check(lib().w4a16_fused_moe_prepared(_stream(x), _ptr(x), _ptr(router_logits.contiguous()), T,
                                         K, I, E, topk, int(renormalize), _ptr(w13.buffer),
                                         _ptr(w2.buffer), G, block_m, _ptr(workspace),
                                         workspace.numel(), _ptr(out)))
    return out


# ------------------------------------------------------------------ kernel level (reference names)

def w4a16_gptq_gemm_typed(a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr, m_size, n_size,
                          k_size, group_size, stride_am, stride_ak, stride_qwk, stride_qwn,
                          stride_sk, stride_sn, stride_qzk, stride_qzn, stride_cm, stride_cn,
                          stream=None):
    """Reference parameter list (w4a16_gptq_gemm_typed.rs:110-128); tensors or raw pointers."""
    st = stream if stream is not None else _stream(a_ptr if isinstance(a_ptr, torch.Tensor) else None)
    args = [_p(a_ptr), _p(qweight_ptr), _p(scales_ptr), _p(qzeros_ptr), _p(c_ptr)]
    check(lib().w4a16_gptq_gemm_typed(st, *args, m_size, n_size, k_size, group_size, stride_am,
                                      stride_ak, stride_qwk, stride_qwn, stride_sk, stride_sn,
                                      stride_qzk, stride_qzn, stride_cm, stride_cn))


def awq_gemm_int4_typed(a_ptr, qweight_ptr, scales_ptr, qzeros_ptr, c_ptr, m_size, n_size,
                        k_size, group_size, stride_am, stride_ak, stride_qwk, stride_qwn,
                        stride_sk, stride_sn, stride_qzk, stride_qzn, stride_cm, stride_cn,
                        stream=None):
    """Reference parameter list (awq_gemm_int4_typed.rs:96-114); tensors or raw pointers."""
    st = stream if stream is not None else _stream(a_ptr if isinstance(a_ptr, torch.Tensor) else None)
    args = [_p(a_ptr), _p(qweight_ptr), _p(scales_ptr), _p(qzeros_ptr), _p(c_ptr)]
    check(lib().awq_gemm_int4_typed(st, *args, m_size, n_size, k_size, group_size, stride_am,
                                    stride_ak, stride_qwk, stride_qwn, stride_sk, stride_sn,
                                    stride_qzk, stride_qzn, stride_cm, stride_cn))


def dequant_int4_to_fp16(qweight, scales, qzeros, output, k_dim, n_dim, group_size, n_div_8,
                         stream=None):
    """ferrum_dequant_int4.rs:27-37: output[n*K + k], zero = nibble (no +1)."""
    st = stream if stream is not None else _stream(qweight if isinstance(qweight, torch.Tensor) else None)
    check(lib().dequant_int4_to_fp16(st, _p(qweight), _p(scales), _p(qzeros), _p(output), k_dim,
                                     n_dim, group_size, n_div_8))


def dequant_int4_sym_to_fp16(qweight, scales, output, k_dim, n_dim, group_size, stream=None):
    """ferrum_dequant_int4_sym.rs:24-31: output[n*K + k], zero = 8."""
    st = stream if stream is not None else _stream(qweight if isinstance(qweight, torch.Tensor) else None)
    check(lib().dequant_int4_sym_to_fp16(st, _p(qweight), _p(scales), _p(output), k_dim, n_dim,
                                         group_size))


def _p(t):
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return ctypes.c_void_p(t.data_ptr())
    return ctypes.c_void_p(int(t))


# ------------------------------------------------------------------ DeviceRuntime mirror

class KernelArg(ctypes.Structure):
    """hiprt_arg: the tagged union for KernelArg{I32,U32,I64,F32,DevicePtr,Bytes}."""

    class _V(ctypes.Union):
        _fields_ = [("i32", ctypes.c_int32), ("u32", ctypes.c_uint32), ("i64", ctypes.c_int64),
                    ("f32", ctypes.c_float), ("device_ptr", ctypes.c_uint64),
                    ("bytes", ctypes.c_void_p)]

    _fields_ = [("kind", ctypes.c_int32), ("size", ctypes.c_uint32), ("v", _V)]

    I32, U32, I64, F32, DEVICE_PTR, BYTES = range(6)

    @classmethod
    def i32(cls, v):
        a = cls(); a.kind = cls.I32; a.v.i32 = v; return a

    @classmethod
    def u32(cls, v):
        a = cls(); a.kind = cls.U32; a.v.u32 = v; return a

    @classmethod
    def i64(cls, v):
        a = cls(); a.kind = cls.I64; a.v.i64 = v; return a

    @classmethod
    def f32(cls, v):
        a = cls(); a.kind = cls.F32; a.v.f32 = v; return a

    @classmethod
    def ptr(cls, v):
        a = cls(); a.kind = cls.DEVICE_PTR
        a.v.device_ptr = v.data_ptr() if isinstance(v, torch.Tensor) else int(v)
        return a


class HipRuntime:
    """DeviceRuntime (crates/triton-runtime/src/lib.rs:64-85) over hiprt_*."""

    def __init__(self, device: int = 0):
        self._ctx = ctypes.c_void_p()
        check(lib().hiprt_create(device, ctypes.byref(self._ctx)))

    def close(self):
        if self._ctx:
            check(lib().hiprt_destroy(self._ctx))
            self._ctx = ctypes.c_void_p()

    def load_module(self, binary: bytes) -> ctypes.c_void_p:
        buf = ctypes.create_string_buffer(binary, len(binary))
        mod = ctypes.c_void_p()
        check(lib().hiprt_module_load(self._ctx, buf, len(binary), ctypes.byref(mod)))
        return mod

    def unload_module(self, module) -> None:
        check(lib().hiprt_module_unload(module))

    def launch(self, module, kernel_name: str, grid, block, shared_mem_bytes: int, stream,
               args) -> None:
        g = (ctypes.c_uint32 * 3)(*grid)
        b = (ctypes.c_uint32 * 3)(*block)
        arr = (KernelArg * max(1, len(args)))(*args)
        st = stream if stream is not None else _stream()
        check(lib().hiprt_launch(self._ctx, module, kernel_name.encode(), g, b, shared_mem_bytes,
                                 st, arr, len(args)))


def typed_module_bytes() -> bytes:
    with open(HSACO_PATH, "rb") as f:
        return f.read()


def typed_module_meta() -> dict:
    import json
    with open(META_PATH) as f:
        return json.load(f)
