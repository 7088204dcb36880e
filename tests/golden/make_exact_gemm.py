"""Generate exact-arithmetic known answers for the W4A16 GEMM (tests/golden/exact_gemm.npz).

The inputs are chosen so that every dequantised weight, every product and every partial sum
any correct implementation forms is exactly representable in fp32, whatever the order of
accumulation:
  x      = j / 4 with j in {-2..2}                  (fp16 exact, granularity 2^-2)
  scale  = 2^-e with e in {3..6}                    (fp16 exact)
  q, z   = nibbles; w = (q - z) * scale             (|w| <= 2, granularity 2^-6)
  x * w  : granularity 2^-8, |x * w| <= 1; sums over K <= 1024 stay below 2^10 -> at most
           18 significant bits, exact in fp32.
The answer is therefore the exact rational sum, rounded once to fp16 (round to nearest,
ties to even). This script computes it with integer arithmetic only (the sum scaled by 2^8,
an int64 matrix product, then an integer round-to-nearest-even into fp16 bits), so it checks
the oracle and the GPU kernels independently of either. The same bound covers the factored form the GEMV kernels use,
s * (sum x (1024 + q) - (1024 + z) sum x), whose intermediate sums stay below 2^18 units of 2^-2.

Weight layouts follow the reference: GPTQ qweight [K/8, N] with row k in nibble k % 8 and
zero = nibble + 1 (crates/triton-dsl/examples/w4a16_gptq_gemm_typed.rs:15-32, :231-236);
GPTQ symmetric zero = 8 (ferrum_dequant_int4_sym.rs:60); AWQ qweight [K, N/8] with column n
in nibble [0,4,1,5,2,6,3,7][n % 8] and zero = nibble (awq_gemm_int4_typed.rs:26-31, :203-205).
Act-order cases use g_idx = a permutation of repeat(0..K/G-1, G).

Run: python tests/golden/make_exact_gemm.py   (writes exact_gemm.npz next to this file)
"""
from __future__ import annotations

import os
import random

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
AWQ_SLOT = [0, 4, 1, 5, 2, 6, 3, 7]   # nibble slot of column n % 8 in an AWQ word

# (name, fmt, M, K, N, G, act_order) -- fmt: 0 GPTQ (+1 zeros), 1 GPTQ symmetric, 2 AWQ.
# Shapes chosen so that every kernel regime of w4a16_gemm is exercised (see test_golden.py).
CASES = [
    ("awq_m1_k512_n256", 2, 1, 512, 256, 128, False),       # VALU GEMV, split K
    ("gptq_m1_k512_n256", 0, 1, 512, 256, 128, False),      # VALU GEMV (GPTQ), split K
    ("sym_m3_k512_n128", 1, 3, 512, 128, 128, False),       # VALU GEMV, M = 3
    ("awq_m8_k512_n256", 2, 8, 512, 256, 128, False),       # matrix-core GEMV, split K
    ("gptq_m16_k512_n256", 0, 16, 512, 256, 128, False),    # small-batch MFMA
    ("awq_m24_k512_n256", 2, 24, 512, 256, 64, False),      # small-batch MFMA (AWQ)
    ("gptq_ao_m16_k512_n256", 0, 16, 512, 256, 128, True),  # small-batch, act-order
    ("gptq_m128_k256_n256", 0, 128, 256, 256, 128, False),  # prefill
    ("awq_m96_k256_n384", 2, 96, 256, 384, 128, False),     # prefill (128-wide tiles)
    ("awq_m5_k384_n200", 2, 5, 384, 200, 128, False),       # generic strided kernel
    ("awq_m6_k1024_n256", 2, 6, 1024, 256, 128, False),     # matrix-core GEMV, 1024-row tile
]


def f16_bits_of_quarter(j: int) -> int:
    """fp16 bit pattern of j / 4 for j in -2..2 (exact)."""
    return int(np.float16(j / 4.0).view(np.uint16))


def f16_bits_rne(num: int, den_log2: int) -> int:
    """fp16 bits of num / 2^den_log2, rounded to nearest-even, with integer arithmetic only
    (normal and subnormal results; |value| < 65504 here)."""
    if num == 0:
        return 0
    sign = 0x8000 if num < 0 else 0
    a = abs(num)
    # value = a * 2^-d; find exponent E with 2^E <= value < 2^(E+1)
    e = a.bit_length() - 1 - den_log2
    if e < -14:
        e = -14                             # subnormal range: fixed exponent, no hidden bit
    # significand with 10 fraction bits: m = value * 2^(10 - e), rounded RNE
    shift = den_log2 - (10 - e)              # m = a / 2^shift
    if shift <= 0:
        m = a << (-shift)
    else:
        q, r = divmod(a, 1 << shift)
        half = 1 << (shift - 1)
        m = q + (1 if (r > half or (r == half and (q & 1))) else 0)
    if m >= 2048:                           # rounding carried into the next binade
        m >>= 1
        e += 1
    if m >= 1024:
        bits = ((e + 15) << 10) | (m - 1024)
    else:
        bits = m                             # subnormal
    assert bits < 0x7C00
    return sign | bits


def make_case(fmt, M, K, N, G, act_order, rng):
    groups = K // G
    xj = [[rng.randint(-2, 2) for _ in range(K)] for _ in range(M)]          # x = j / 4
    q = [[rng.randint(0, 15) for _ in range(N)] for _ in range(K)]            # nibbles
    zn = [[rng.randint(0, 15) for _ in range(N)] for _ in range(groups)]     # stored zeros
    se = [[rng.randint(3, 6) for _ in range(N)] for _ in range(groups)]      # scale = 2^-se
    if act_order:
        g_idx = [k // G for k in range(K)]
        rng.shuffle(g_idx)
    else:
        g_idx = None

    def zero(g, n):
        if fmt == 1:
            return 8
        return zn[g][n] + (1 if fmt == 0 else 0)

    # exact result: sum_k (j/4) * (q - z) * 2^-se = (1/2^8) * sum_k j * (q - z) * 2^(6 - se),
    # an integer matrix product (int64, exact: |sum| <= 1024 * 2 * 16 * 8)
    w_int = np.zeros((K, N), dtype=np.int64)
    for k in range(K):
        g = g_idx[k] if act_order else k // G
        for n in range(N):
            w_int[k, n] = (q[k][n] - zero(g, n)) * (1 << (6 - se[g][n]))
    acc = np.array(xj, dtype=np.int64) @ w_int
    out_bits = np.zeros((M, N), dtype=np.uint16)
    for m in range(M):
        for n in range(N):
            out_bits[m, n] = f16_bits_rne(int(acc[m, n]), 8)

    x = np.array([[f16_bits_of_quarter(j) for j in row] for row in xj], dtype=np.uint16)
    scales = np.array([[int(np.float16(2.0 ** -e).view(np.uint16)) for e in row] for row in se],
                      dtype=np.uint16)
    if fmt == 2:
        qw = np.zeros((K, N // 8), dtype=np.uint32)
        for k in range(K):
            for n in range(N):
                qw[k, n // 8] |= np.uint32(q[k][n] << (4 * AWQ_SLOT[n % 8]))
        qz = np.zeros((groups, N // 8), dtype=np.uint32)
        for g in range(groups):
            for n in range(N):
                qz[g, n // 8] |= np.uint32(zn[g][n] << (4 * AWQ_SLOT[n % 8]))
    else:
        qw = np.zeros((K // 8, N), dtype=np.uint32)
        for k in range(K):
            for n in range(N):
                qw[k // 8, n] |= np.uint32(q[k][n] << (4 * (k % 8)))
        qz = np.zeros((groups, N // 8), dtype=np.uint32)
        for g in range(groups):
            for n in range(N):
                qz[g, n // 8] |= np.uint32(zn[g][n] << (4 * (n % 8)))
    gi = np.array(g_idx if act_order else [], dtype=np.int32)
    return x, qw.view(np.int32), scales, qz.view(np.int32), gi, out_bits


def main():
    rng = random.Random(0x5EED60D)
    arrays = {}
    for name, fmt, M, K, N, G, ao in CASES:
        x, qw, sc, qz, gi, out = make_case(fmt, M, K, N, G, ao, rng)
        meta = np.array([fmt, M, K, N, G, int(ao)], dtype=np.int32)
        for key, val in (("meta", meta), ("x", x), ("qweight", qw), ("scales", sc),
                         ("qzeros", qz), ("g_idx", gi), ("out", out)):
            arrays[f"{name}/{key}"] = val
    path = os.path.join(HERE, "exact_gemm.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
