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


# ------------------------------------------------------------------ prepared layout

PREP_SLOT = tuple((i >> 1) | ((i & 1) << 2) for i in range(8))   # nibble slot of row i of a word


def prepared_table_rows(G: int) -> int:
    """Table rows per 128-row block: the block's groups (G = 32, 64) or its one group."""
    return 128 // G if G < 128 else 1


def prepared_table_words(K: int, G: int) -> int:
    return ((K // 128) * prepared_table_rows(G) * 16 + 63) // 64 * 64


def prepared_strip_bytes(K: int, G: int) -> int:
    return 4 * prepared_table_words(K, G) + K * 8


def prepared_layout(q: np.ndarray, zint: np.ndarray, scales: np.ndarray, G: int) -> np.ndarray:
    """The prepared layout (include/w4a16.h, w4a16_prepare_layout) written from the integer
    matrices: q [K, N] nibbles, zint [K/G, N] full zero points, scales fp16 [K/G, N].
    Strip s: the table, for each block kb of 128 rows R rows r of 16 entries, entry (kb, r, c) =
    fp16 bits of scales[g, 16 s + c] | zint[g, 16 s + c] << 16 with g = 128 kb // G + r, padded
    to 256 bytes; then the blocks, 64 lanes x 4 words, lane l = column 16 s + l % 16, word w =
    rows 128 kb + 32 (l // 16) + 8 w + [0, 8), row i in nibble slot PREP_SLOT[i].
    Returns uint8 [N/16 * strip bytes]."""
    K, N = q.shape
    R = prepared_table_rows(G)
    tw = prepared_table_words(K, G)
    out = np.zeros((N // 16, tw + K * 2), dtype=np.uint32)
    ent = scales.view(np.uint16).astype(np.uint32) | (zint.astype(np.uint32) << np.uint32(16))
    g = (np.arange(K // 128)[:, None] * 128 // G + np.arange(R)[None, :]).reshape(-1)   # [kb*R + r]
    tab = ent[g]                                                   # [blocks*R, N]
    out[:, :len(g) * 16] = tab.reshape(len(g), N // 16, 16).transpose(1, 0, 2).reshape(N // 16, -1)
    # q as [strip, kb, h, w, i, col]: rows 128 kb + 32 h + 8 w + i, column 16 s + col
    qq = q.astype(np.uint32).reshape(K // 128, 4, 4, 8, N // 16, 16).transpose(4, 0, 1, 2, 3, 5)
    words = np.zeros(qq.shape[:4] + (16,), dtype=np.uint32)   # [s, kb, h, w, col]
    for i in range(8):
        words |= qq[:, :, :, :, i, :] << np.uint32(4 * PREP_SLOT[i])
    # lane l = 16 h + col, word w at l * 4 + w: order [s, kb, h, col, w]
    out[:, tw:] = words.transpose(0, 1, 2, 4, 3).reshape(N // 16, K * 2)
    return out.view(np.uint8).reshape(-1)
