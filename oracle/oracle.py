"""ctypes binding of the CPU oracle (liborc_w4a16.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only to check or to time the CPU baseline; the HIP product path never
calls it. Arrays are numpy; fp16 values travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc_w4a16.so")

FMT_GPTQ, FMT_GPTQ_SYM, FMT_AWQ = 0, 1, 2

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE, "CC=gcc"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_f16_array.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_f16_to_f32_array.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_awq_slot.argtypes = [_I]
    L.orc_nibble.argtypes = [ctypes.c_int32, _I]
    L.orc_qweight_at.argtypes = [_I, _P, _I, _I, _I, _I]
    L.orc_zero_at.argtypes = [_I, _P, _I, _I, _I, _I]
    L.orc_dequant.argtypes = [_I, _P, _P, _P, _P, _I, _I, _I, _I, _P]
    L.orc_dequant_transposed.argtypes = [_I, _P, _P, _P, _P, _I, _I, _I, _I, _P]
    L.orc_gemm_f16.argtypes = [_P, _P, _I, _I, _I, _I, _P, _P]
    L.orc_w4a16_gemm.argtypes = [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P]
    L.orc_w4a16_gemm_rows.argtypes = [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P]
    L.orc_moe_route.argtypes = [_P, _I, _I, _I, _P, _P]
    L.orc_moe_align.argtypes = [_P, _I, _I, _I, _I, _P, _P]
    L.orc_moe_align.restype = _I
    L.orc_moe_forward.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]
    L.orc_silu_mul_f16.restype = ctypes.c_uint16
    L.orc_silu_mul_f16.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
    L.orc_silu_mul_f32.restype = ctypes.c_float
    L.orc_silu_mul_f32.argtypes = [ctypes.c_float, ctypes.c_float]
    L.orc_silu_mul_f32_rows.restype = None
    L.orc_silu_mul_f32_rows.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_bf16_array.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_bf16_to_f32_array.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_dequant_bf16.argtypes = [_I, _P, _P, _P, _P, _I, _I, _I, _I, _P]
    L.orc_dequant_transposed_bf16.argtypes = [_I, _P, _P, _P, _P, _I, _I, _I, _I, _P]
    L.orc_w4a16_gemm_bf16.argtypes = [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P]
    L.orc_num_threads.restype = _I
    L.orc_set_num_threads.argtypes = [_I]


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


def _i32(a):
    if a is None:
        return None
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    assert a.dtype == np.int32, a.dtype
    return a


def f32_to_f16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def f16_bits_to_f32(a) -> np.ndarray:
    a = _u16(a)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def f32_to_bf16_bits(a) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values, rounded to nearest even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_ptr(a), _ptr(out), a.size)
    return out


def bf16_bits_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def dequant_bf16(fmt, qweight, scales_bits, qzeros, K, N, G, g_idx=None, zero_offset=1,
                 transposed=False) -> np.ndarray:
    """W as bfloat16 bit patterns (uint16) [K, N] (or [N, K]) from bf16 scale bits."""
    qweight, qzeros, g_idx = _i32(qweight), _i32(qzeros), _i32(g_idx)
    scales = np.ascontiguousarray(scales_bits, dtype=np.uint16)
    out = np.empty((N, K) if transposed else (K, N), dtype=np.uint16)
    fn = lib().orc_dequant_transposed_bf16 if transposed else lib().orc_dequant_bf16
    rc = fn(fmt, _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx), K, N, G,
            zero_offset, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle dequant failed rc={rc}")
    return out


def w4a16_gemm_bf16(fmt, x_bits, qweight, scales_bits, qzeros, K, N, G, g_idx=None,
                    zero_offset=1, acc64=True):
    """(out bf16 bits [M, N], unrounded f32 sums) of the bfloat16 instantiation."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    qweight, qzeros, g_idx = _i32(qweight), _i32(qzeros), _i32(g_idx)
    scales = np.ascontiguousarray(scales_bits, dtype=np.uint16)
    M = x.shape[0]
    out = np.empty((M, N), dtype=np.uint16)
    of = np.empty((M, N), dtype=np.float32)
    rc = lib().orc_w4a16_gemm_bf16(fmt, _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros),
                                   _ptr(g_idx), M, N, K, G, zero_offset, 1 if acc64 else 0,
                                   _ptr(out), _ptr(of))
    if rc != 0:
        raise ValueError(f"oracle gemm failed rc={rc}")
    return out, of


def awq_slot(n: int) -> int:
    return lib().orc_awq_slot(n)


def nibble(word: int, slot: int) -> int:
    return lib().orc_nibble(ctypes.c_int32(np.int32(np.uint32(word & 0xFFFFFFFF)).item()), slot)


def qweight_at(fmt, qweight, K, N, k, n) -> int:
    qweight = _i32(qweight)
    return lib().orc_qweight_at(fmt, _ptr(qweight), K, N, k, n)


def zero_at(fmt, qzeros, N, g, n, zero_offset=1) -> int:
    qzeros = _i32(qzeros)
    return lib().orc_zero_at(fmt, _ptr(qzeros), N, g, n, zero_offset)


def dequant(fmt, qweight, scales, qzeros, K, N, G, g_idx=None, zero_offset=1,
            transposed=False) -> np.ndarray:
    """W16 as float16 array [K, N] (or [N, K] when transposed)."""
    qweight, qzeros, g_idx = _i32(qweight), _i32(qzeros), _i32(g_idx)
    scales = _u16(scales)
    out = np.empty((N, K) if transposed else (K, N), dtype=np.uint16)
    fn = lib().orc_dequant_transposed if transposed else lib().orc_dequant
    rc = fn(fmt, _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx), K, N, G,
            zero_offset, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle dequant failed rc={rc}")
    return out.view(np.float16)


def gemm_f16(x, w16, acc64=True, want_f32=False):
    x, w16 = _u16(x), _u16(w16)
    M, K = x.shape
    K2, N = w16.shape
    assert K == K2
    out = np.empty((M, N), dtype=np.uint16)
    of = np.empty((M, N), dtype=np.float32) if want_f32 else None
    lib().orc_gemm_f16(_ptr(x), _ptr(w16), M, N, K, 1 if acc64 else 0, _ptr(out), _ptr(of))
    return (out.view(np.float16), of) if want_f32 else out.view(np.float16)


def w4a16_gemm(fmt, x, qweight, scales, qzeros, K, N, G, g_idx=None, zero_offset=1,
               acc64=True, want_f32=False):
    x = _u16(x)
    qweight, qzeros, g_idx = _i32(qweight), _i32(qzeros), _i32(g_idx)
    scales = _u16(scales)
    M = x.shape[0]
    out = np.empty((M, N), dtype=np.uint16)
    of = np.empty((M, N), dtype=np.float32) if want_f32 else None
    rc = lib().orc_w4a16_gemm(fmt, _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros),
                              _ptr(g_idx), M, N, K, G, zero_offset, 1 if acc64 else 0,
                              _ptr(out), _ptr(of))
    if rc != 0:
        raise ValueError(f"oracle gemm failed rc={rc}")
    return (out.view(np.float16), of) if want_f32 else out.view(np.float16)


def w4a16_gemm_rows(fmt, x, qweight, scales, qzeros, K, N, G, rows, g_idx=None,
                    zero_offset=1):
    x = _u16(x)
    qweight, qzeros, g_idx = _i32(qweight), _i32(qzeros), _i32(g_idx)
    scales = _u16(scales)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    out = np.empty((rows.size, N), dtype=np.uint16)
    rc = lib().orc_w4a16_gemm_rows(fmt, _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros),
                                   _ptr(g_idx), x.shape[0], N, K, G, zero_offset,
                                   _ptr(rows), rows.size, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle gemm_rows failed rc={rc}")
    return out.view(np.float16)


def moe_route(logits, topk):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, topk), dtype=np.int32)
    w = np.empty((T, topk), dtype=np.float32)
    lib().orc_moe_route(_ptr(logits), T, E, topk, _ptr(ids), _ptr(w))
    return ids, w


def moe_align(ids, E, block_m):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, topk = ids.shape
    cap = T * topk + E * (block_m - 1)
    sorted_ids = np.empty(cap, dtype=np.int32)
    expert_ids = np.empty((cap + block_m - 1) // block_m, dtype=np.int32)
    n = lib().orc_moe_align(_ptr(ids), T, topk, E, block_m, _ptr(sorted_ids), _ptr(expert_ids))
    return sorted_ids[:n].copy(), expert_ids[: n // block_m].copy(), n


def moe_forward(x, ids, weights, w13_list, w2_list, inter=None):
    """y[T, K] from dequantised per-expert w13 [K, 2I] and w2 [I, K] (float16 arrays).
    Experts no token selects may be placeholders when `inter` (I) is given."""
    x = _u16(x)
    T, K = x.shape
    E = len(w13_list)
    I = inter if inter is not None else w2_list[0].shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    topk = ids.shape[1]
    w13 = [_u16(a) for a in w13_list]
    w2 = [_u16(a) for a in w2_list]
    p13 = (ctypes.c_void_p * E)(*[a.ctypes.data for a in w13])
    p2 = (ctypes.c_void_p * E)(*[a.ctypes.data for a in w2])
    y = np.empty((T, K), dtype=np.uint16)
    lib().orc_moe_forward(_ptr(x), T, K, I, E, topk, _ptr(ids), _ptr(weights),
                          ctypes.cast(p13, ctypes.c_void_p), ctypes.cast(p2, ctypes.c_void_p),
                          _ptr(y))
    return y.view(np.float16)


def silu_mul_f16(g, u) -> np.ndarray:
    g, u = _u16(g).ravel(), _u16(u).ravel()
    L = lib()
    return np.array([L.orc_silu_mul_f16(int(a), int(b)) for a, b in zip(g, u)],
                    dtype=np.uint16).view(np.float16)


def silu_mul_f32_rows(gate_up, inter, total) -> np.ndarray:
    """fused_silu_mul_interleaved_f32 over a flat float32 buffer (elementwise.rs:214-250)."""
    gu = np.ascontiguousarray(gate_up, dtype=np.float32).ravel()
    out = np.empty(total, dtype=np.float32)
    lib().orc_silu_mul_f32_rows(_ptr(gu), _ptr(out), int(inter), int(total))
    return out


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)
