"""Pins the oracle's bfloat16 instantiation (CPU only).

The reference kernels are generic over the element type and name bf16
(w4a16_gptq_gemm_typed.rs:65-67): the weight is as_t::<bf16>(f32(q - z) * f32(s)) and the
output as_t::<bf16>(f32 accumulator), with as_t = truncf, round to nearest even. The checks
compare the oracle against torch's own float32 -> bfloat16 conversion (an independent
implementation), against the closed form bits << 16 for the widening, and against a float64
matmul built from the integer matrices.
"""
import numpy as np
import pytest
import torch

import synth
from synth import Problem

GPTQ, SYM, AWQ = 0, 1, 2


def torch_bf16_bits(f32: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(f32, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_bf16_to_f32_all_65536(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.bf16_bits_to_f32(bits).view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_f32_to_bf16_matches_torch_on_random_and_edge_patterns(orc):
    g = np.random.default_rng(11)
    rnd = g.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    hi = g.integers(0, 2 ** 16, size=4096, dtype=np.uint64).astype(np.uint32) << 16
    edges = np.concatenate([
        hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi,          # ties (both parities) and neighbours
        np.array([0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0xFF7FFFFF,   # near the largest finite
                  0x00000001, 0x00008000, 0x00018000, 0x807FFFFF,   # subnormals
                  0x00000000, 0x80000000, 0x7F800000, 0xFF800000], dtype=np.uint32),
    ])
    pats = np.concatenate([rnd, edges])
    f = pats.view(np.float32)
    got = orc.f32_to_bf16_bits(f)
    want = torch_bf16_bits(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN stays NaN (exponent all ones, mantissa non-zero), sign kept
    g16 = got[nan].astype(np.uint32)
    assert np.all(((g16 >> 7) & 0xFF) == 0xFF) and np.all((g16 & 0x7F) != 0)
    assert np.array_equal(g16 >> 15, (pats[nan] >> 31))


def test_dequant_bf16_exhaustive_closed_form(orc):
    """Every nibble x every zero point (GPTQ offsets 0 and 1) x every bfloat16 scale in
    [0.002, 0.02]: W = RNE_bf16((q - z) * s), with the product exact in f32."""
    lo, hi = torch_bf16_bits(np.float32([0.002, 0.02]))
    sc_bits = np.arange(lo, hi + 1, dtype=np.uint16)
    S = sc_bits.size
    assert S > 400
    Np = 8 * ((S + 7) // 8)
    scales_bits = np.resize(sc_bits, Np).reshape(1, Np)
    s32 = orc.bf16_bits_to_f32(scales_bits)
    for z in range(0, 17):
        for zero_offset in (1, 0):
            if not (zero_offset <= z <= 15 + zero_offset):
                continue
            q = np.tile(np.arange(8, dtype=np.int32)[:, None], (1, Np))
            for half in (0, 8):
                qq = q + half
                qweight = synth.pack_gptq_qweight(qq)
                zq = np.full((1, Np), z - zero_offset, dtype=np.int32)
                qzeros = synth.pack_along_n(zq, awq=False)
                got = orc.dequant_bf16(GPTQ, qweight, scales_bits, qzeros, 8, Np, 8,
                                       zero_offset=zero_offset)
                want = torch_bf16_bits((qq - z).astype(np.float32) * s32)
                assert np.array_equal(got, want), (z, zero_offset)


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
def test_dequant_bf16_matches_integer_definition(orc, fmt):
    p = Problem(fmt, M=1, K=256, N=64, G=64, seed=40 + fmt)
    s_bits = torch_bf16_bits(p.scales.astype(np.float32))
    s32 = orc.bf16_bits_to_f32(s_bits)
    g = np.arange(p.K) // p.G
    want = torch_bf16_bits((p.q - p.zero_int()[g]).astype(np.float32) * s32[g])
    got = orc.dequant_bf16(fmt, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G)
    assert np.array_equal(got, want)
    t = orc.dequant_bf16(fmt, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G, transposed=True)
    assert np.array_equal(t, want.T)


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
def test_gemm_bf16_brute_force_f64(orc, fmt):
    """out = RNE_bf16(sum_k x * W) with x and W bfloat16: float64 matmul of the integer
    definition, rounded once."""
    p = Problem(fmt, M=5, K=384, N=48, G=128, seed=50 + fmt)
    x_bits = torch_bf16_bits(p.x.astype(np.float32))
    s_bits = torch_bf16_bits(p.scales.astype(np.float32))
    g = np.arange(p.K) // p.G
    w = orc.bf16_bits_to_f32(torch_bf16_bits(
        (p.q - p.zero_int()[g]).astype(np.float32) * orc.bf16_bits_to_f32(s_bits)[g]))
    ref = orc.bf16_bits_to_f32(x_bits).astype(np.float64) @ w.astype(np.float64)
    out, f32 = orc.w4a16_gemm_bf16(fmt, x_bits, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G)
    assert np.array_equal(f32, ref.astype(np.float32))
    assert np.array_equal(out, torch_bf16_bits(ref.astype(np.float32)))


def test_gemm_bf16_act_order_equals_permuted_plain(orc):
    """g_idx: the act-order product equals the plain product over the rows grouped by g_idx
    (rows of x and of the unpacked weights permuted together)."""
    p = Problem(GPTQ, M=3, K=512, N=32, G=128, seed=60, act_order=True)
    x_bits = torch_bf16_bits(p.x.astype(np.float32))
    s_bits = torch_bf16_bits(p.scales.astype(np.float32))
    out, f32 = orc.w4a16_gemm_bf16(GPTQ, x_bits, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G,
                                   g_idx=p.g_idx)
    w = orc.bf16_bits_to_f32(orc.dequant_bf16(GPTQ, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G,
                                              g_idx=p.g_idx))
    # W row k uses group g_idx[k]: recompute it from the definition
    want_w = torch_bf16_bits((p.q - p.zero_int()[p.g_idx]).astype(np.float32)
                             * orc.bf16_bits_to_f32(s_bits)[p.g_idx])
    assert np.array_equal(torch_bf16_bits(w), want_w)
    ref = orc.bf16_bits_to_f32(x_bits).astype(np.float64) @ w.astype(np.float64)
    assert np.array_equal(f32, ref.astype(np.float32))
