"""Seeded synthetic inputs for the W4A16 configs, plus int4 packing.

Packing is written here independently of any unpacking code (it goes from
integer nibbles to packed int32 words), so the oracle's and the HIP kernels'
unpackers can be checked against it.

Value distributions follow the benchmark configs: x ~ N(0,1) in fp16, nibbles
uniform in 0..15, scales uniform in [0.002, 0.02] rounded to fp16, g_idx a seeded
permutation of repeat(0..K/G-1, G). Seeds are 0x5EED0000 + config index.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x5EED0000

# AWQ pack order: slot i of a word holds column AWQ_PACK_ORDER[i] of its 8-column group
# (the AWQ benchmark config). Reading column n back therefore uses slot AWQ_UNPACK_SLOT[n],
# the inverse permutation [0,4,1,5,2,6,3,7]
# (crates/triton-dsl/examples/awq_gemm_int4_typed.rs:26-31).
AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_UNPACK_SLOT = tuple(AWQ_PACK_ORDER.index(n) for n in range(8))


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def pack_gptq_qweight(q: np.ndarray) -> np.ndarray:
    """q [K, N] ints 0..15 -> int32 [K/8, N], row k in slot k%8 (straight)."""
    K, N = q.shape
    assert K % 8 == 0
    q = q.astype(np.uint32).reshape(K // 8, 8, N)
    w = np.zeros((K // 8, N), dtype=np.uint32)
    for s in range(8):
        w |= q[:, s, :] << np.uint32(4 * s)
    return w.view(np.int32)


def pack_along_n(q: np.ndarray, awq: bool) -> np.ndarray:
    """q [R, N] ints 0..15 -> int32 [R, N/8] packed along N.

    GPTQ (qzeros): column n in slot n%8. AWQ (qweight and qzeros): slot i holds
    column AWQ_PACK_ORDER[i]."""
    R, N = q.shape
    assert N % 8 == 0
    q = q.astype(np.uint32).reshape(R, N // 8, 8)
    w = np.zeros((R, N // 8), dtype=np.uint32)
    for s in range(8):
        col = AWQ_PACK_ORDER[s] if awq else s
        w |= q[:, :, col] << np.uint32(4 * s)
    return w.view(np.int32)


def rand_x(g: np.random.Generator, M: int, K: int) -> np.ndarray:
    return g.standard_normal((M, K), dtype=np.float32).astype(np.float16)


def rand_scales(g: np.random.Generator, ngroups: int, N: int) -> np.ndarray:
    return g.uniform(0.002, 0.02, size=(ngroups, N)).astype(np.float32).astype(np.float16)


def rand_nibbles(g: np.random.Generator, shape) -> np.ndarray:
    return g.integers(0, 16, size=shape, dtype=np.int32)


def act_order_gidx(g: np.random.Generator, K: int, G: int) -> np.ndarray:
    """Seeded permutation of repeat(0..K/G-1, G) (the act-order benchmark config)."""
    base = np.repeat(np.arange(K // G, dtype=np.int32), G)
    return g.permutation(base).astype(np.int32)


class Problem:
    """One W4A16 GEMM problem: packed weights plus the integer matrices they came from."""

    def __init__(self, fmt: int, M: int, K: int, N: int, G: int = 128, seed: int = 0,
                 act_order: bool = False, zero_offset: int = 1):
        from_fmt = {0: "gptq", 1: "gptq_sym", 2: "awq"}
        self.fmt, self.M, self.K, self.N, self.G = fmt, M, K, N, G
        self.kind = from_fmt[fmt]
        self.zero_offset = zero_offset
        g = rng(seed)
        self.x = rand_x(g, M, K)
        self.q = rand_nibbles(g, (K, N))
        ng = K // G
        self.scales = rand_scales(g, ng, N)
        self.zq = rand_nibbles(g, (ng, N))
        if fmt == 2:
            self.qweight = pack_along_n(self.q, awq=True)
            self.qzeros = pack_along_n(self.zq, awq=True)
        else:
            self.qweight = pack_gptq_qweight(self.q)
            self.qzeros = pack_along_n(self.zq, awq=False) if fmt == 0 else None
        self.g_idx = act_order_gidx(g, K, G) if act_order else None

    def zero_int(self) -> np.ndarray:
        """Integer zero points [K/G, N] implied by the format."""
        if self.fmt == 1:
            return np.full(self.zq.shape, 8, dtype=np.int32)
        if self.fmt == 0:
            return self.zq + self.zero_offset
        return self.zq
