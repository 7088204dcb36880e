"""Pins the CPU oracle before anything is checked against it.

The reference holds no numeric test, golden vector or fixture for this path (its only
test, crates/triton-dsl/tests/proc_macro_awq_gemm.rs, asserts MLIR text). Each oracle
function is therefore pinned by known answers, library routines (numpy's IEEE
binary16 conversion and float64 matmul), closed forms and invariants, chosen so that
a dropped term, a wrong sign, a wrong nibble order or a transposed operand fails.
"""
import numpy as np
import pytest

import synth
from synth import AWQ_UNPACK_SLOT, Problem

GPTQ, SYM, AWQ = 0, 1, 2


# ---------------------------------------------------------------- fp16 conversion

def test_f16_to_f32_all_65536(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _check_f32_to_f16(orc, f32):
    got = orc.f32_to_f16_bits(f32)
    with np.errstate(over="ignore"):
        want = f32.astype(np.float16).view(np.uint16)
    nan = np.isnan(f32)
    assert np.array_equal(got[~nan], want[~nan]), np.nonzero(got[~nan] != want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_f32_to_f16_ties_and_neighbours(orc):
    # every finite f16, the exact midpoints between neighbours (round-half-even cases),
    # and the f32 values one ulp either side of each midpoint
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2.0
    mids32 = mids.astype(np.float32)
    up = np.nextafter(mids32, np.float32(np.inf))
    dn = np.nextafter(mids32, np.float32(0))
    top = np.array([65504.0, 65519.99, 65520.0, 65536.0, 1e30, np.inf, -np.inf, np.nan,
                    2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 1e-30, 0.0,
                    -0.0], dtype=np.float32)
    for arr in (h.astype(np.float32), mids32, up, dn, top):
        _check_f32_to_f16(orc, np.concatenate([arr, -arr]))


def test_f32_to_f16_random_bit_patterns(orc):
    g = np.random.default_rng(1)
    bits = g.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    _check_f32_to_f16(orc, bits.view(np.float32))
    # concentrated on the f16 range, where the mantissa rounding matters
    _check_f32_to_f16(orc, (g.standard_normal(2_000_000) * 100).astype(np.float32))


# ---------------------------------------------------------------- nibble order

def test_known_answer_nibble_order(orc):
    # word 0x76543210 holds value s in slot s.
    w = np.array([0x76543210], dtype=np.uint32).view(np.int32)
    # GPTQ packs 8 K-rows per word in straight order (w4a16_gptq_gemm_typed.rs:175-180)
    gptq_rows = [orc.qweight_at(GPTQ, w.reshape(1, 1), 8, 1, k, 0) for k in range(8)]
    assert gptq_rows == [0, 1, 2, 3, 4, 5, 6, 7]
    # AWQ packs 8 N-columns per word; column n reads slot [0,4,1,5,2,6,3,7][n]
    # (awq_gemm_int4_typed.rs:26-31, 139-151)
    awq_cols = [orc.qweight_at(AWQ, w.reshape(1, 1), 1, 8, 0, n) for n in range(8)]
    assert awq_cols == [0, 4, 1, 5, 2, 6, 3, 7]
    w2 = np.array([0xFEDCBA98], dtype=np.uint32).view(np.int32).reshape(1, 1)
    assert [orc.qweight_at(AWQ, w2, 1, 8, 0, n) for n in range(8)] == [8, 12, 9, 13, 10, 14, 11, 15]
    assert [orc.qweight_at(GPTQ, w2, 8, 1, k, 0) for k in range(8)] == list(range(8, 16))
    # the constants the reference's structural test demands for the AWQ remap:
    # n%8 via 8, nibble mask 15, (n%8)/2 and (n%8)%2 via 2, *4 (proc_macro_awq_gemm.rs:262-324)
    assert [orc.awq_slot(n) for n in range(16)] == [(n % 8) // 2 + ((n % 8) % 2) * 4 for n in range(16)]
    assert tuple(orc.awq_slot(n) for n in range(8)) == AWQ_UNPACK_SLOT
    # logical (not arithmetic) shift: the top nibble of a negative word is 0..15
    neg = np.array([0xF0000000], dtype=np.uint32).view(np.int32).reshape(1, 1)
    assert orc.qweight_at(GPTQ, neg, 8, 1, 7, 0) == 15


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
def test_pack_unpack_roundtrip(orc, fmt):
    p = Problem(fmt, M=1, K=256, N=64, G=128, seed=3)
    deq_int = np.array([[orc.qweight_at(fmt, p.qweight, p.K, p.N, k, n) for n in range(p.N)]
                        for k in range(0, p.K, 7)])
    assert np.array_equal(deq_int, p.q[::7])
    zeros = np.array([[orc.zero_at(fmt, p.qzeros, p.N, g, n, 1) for n in range(p.N)]
                      for g in range(p.K // p.G)])
    assert np.array_equal(zeros, p.zero_int())


# ---------------------------------------------------------------- dequant

def test_dequant_exhaustive_closed_form(orc):
    """Every (q, z) with every fp16 scale in [0.002, 0.02]: W16 = RNE_f16((q - z) * s).

    Every zero point 0..16 (GPTQ offsets 0 and 1) x all 16 nibbles x every fp16 scale.
    The expectation uses numpy's binary16 rounding of the exact f32 product."""
    lo = np.float16(0.002).view(np.uint16)
    hi = np.float16(0.02).view(np.uint16)
    sc_bits = np.arange(lo, hi + 1, dtype=np.uint16)
    sc = sc_bits.view(np.float16)
    assert sc.size > 3000
    S = sc.size
    # K = 8 rows (one GPTQ word), N = S columns, G = 8: scales row 0 = all scales.
    for z in range(0, 17):
        for fmt, zero_offset in ((GPTQ, 1), (GPTQ, 0)):
            if fmt == GPTQ and not (zero_offset <= z <= 15 + zero_offset):
                continue
            q = np.tile(np.arange(8, dtype=np.int32)[:, None], (1, 8 * ((S + 7) // 8)))
            for half in (0, 8):
                qq = q + half
                Np = qq.shape[1]
                qweight = synth.pack_gptq_qweight(qq)
                scales = np.resize(sc, Np).reshape(1, Np)
                zq = np.full((1, Np), z - zero_offset, dtype=np.int32)
                qzeros = synth.pack_along_n(zq, awq=False)
                got = orc.dequant(fmt, qweight, scales, qzeros, 8, Np, 8, zero_offset=zero_offset)
                want = ((qq - z).astype(np.float32) * scales.astype(np.float32)).astype(np.float16)
                assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), (z, zero_offset)
                # invariant: one correctly rounded fp16 multiply of fp16(q - z) * s gives the
                # same bits, because (q - z) * s is exact in f32
                want16 = (qq - z).astype(np.float16) * scales
                assert np.array_equal(want16.view(np.uint16), want.view(np.uint16))


def test_zero_conventions(orc):
    p = Problem(GPTQ, M=1, K=256, N=64, G=64, seed=5)
    # GPTQ with every stored zero nibble = 7 (+1 => 8) equals the symmetric format
    q7 = np.full(p.zq.shape, 7, dtype=np.int32)
    qz7 = synth.pack_along_n(q7, awq=False)
    a = orc.dequant(GPTQ, p.qweight, p.scales, qz7, p.K, p.N, p.G, zero_offset=1)
    b = orc.dequant(SYM, p.qweight, p.scales, None, p.K, p.N, p.G)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    # offset-0 dequant (ferrum_dequant_int4.rs) with nibble z == offset-1 GEMM with nibble z-1
    zq = np.clip(p.zq, 1, 15)
    a = orc.dequant(GPTQ, p.qweight, p.scales, synth.pack_along_n(zq, False), p.K, p.N, p.G,
                    zero_offset=0)
    b = orc.dequant(GPTQ, p.qweight, p.scales, synth.pack_along_n(zq - 1, False), p.K, p.N,
                    p.G, zero_offset=1)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    # and a +1 actually shifts every weight by one scale step (the term is not dropped)
    c = orc.dequant(GPTQ, p.qweight, p.scales, synth.pack_along_n(zq, False), p.K, p.N, p.G,
                    zero_offset=1)
    diff = a.astype(np.float32) - c.astype(np.float32)
    s_k = np.repeat(p.scales.astype(np.float32), p.G, axis=0)
    # each side is rounded to fp16 once: |err| <= 2 half-ulps at |w| <= 0.32 (ulp 2^-12)
    assert np.allclose(diff, s_k, rtol=0, atol=2.5e-4)


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
def test_dequant_matches_integer_definition(orc, fmt):
    """Compare against the dequant built from the pre-packing integer matrices."""
    p = Problem(fmt, M=1, K=512, N=96, G=128, seed=11)
    got = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G)
    zk = np.repeat(p.zero_int(), p.G, axis=0)
    sk = np.repeat(p.scales.astype(np.float32), p.G, axis=0)
    want = ((p.q - zk).astype(np.float32) * sk).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    t = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, transposed=True)
    assert t.shape == (p.N, p.K)
    assert np.array_equal(t.view(np.uint16), got.T.view(np.uint16))


# ---------------------------------------------------------------- GEMM

@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
def test_gemm_brute_force_f64(orc, fmt):
    p = Problem(fmt, M=3, K=256, N=24, G=128, seed=21)
    w16 = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G)
    want = p.x.astype(np.float64) @ w16.astype(np.float64)
    y64, f64 = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                              acc64=True, want_f32=True)
    assert np.allclose(f64, want, rtol=1e-6, atol=1e-7)
    assert np.array_equal(y64.view(np.uint16), want.astype(np.float32).astype(np.float16).view(np.uint16))
    y32, f32 = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                              acc64=False, want_f32=True)
    assert np.allclose(f32, want, rtol=1e-4, atol=1e-4)
    # operands not transposed: a non-square K x N where the transpose would not even fit
    assert y32.shape == (p.M, p.N)


def test_gemm_closed_forms(orc):
    p = Problem(AWQ, M=4, K=256, N=32, G=128, seed=31)
    w16 = orc.dequant(AWQ, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G)
    # one-hot x selects a row of W16 exactly
    x = np.zeros((4, p.K), dtype=np.float16)
    rows = [0, 7, 128, 255]
    for i, r in enumerate(rows):
        x[i, r] = 1.0
    y = orc.gemm_f16(x, w16)
    assert np.array_equal(y.view(np.uint16), w16[rows].view(np.uint16))
    # scale 1 and (q - z) = c everywhere => y = c * sum(x)
    q = np.full((p.K, p.N), 11, dtype=np.int32)
    zq = np.full((p.K // p.G, p.N), 4, dtype=np.int32)
    ones = np.ones((p.K // p.G, p.N), dtype=np.float16)
    y = orc.w4a16_gemm(AWQ, p.x, synth.pack_along_n(q, True), ones,
                       synth.pack_along_n(zq, True), p.K, p.N, p.G)
    want = (7.0 * p.x.astype(np.float64).sum(axis=1))[:, None] * np.ones((1, p.N))
    assert np.allclose(y.astype(np.float64), want, rtol=1e-3, atol=1e-3)


def test_gemm_rows_sample_equals_full(orc):
    p = Problem(GPTQ, M=16, K=256, N=40, G=64, seed=41)
    full = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G)
    rows = np.array([15, 0, 7], dtype=np.int32)
    part = orc.w4a16_gemm_rows(GPTQ, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, rows)
    assert np.array_equal(part.view(np.uint16), full[rows].view(np.uint16))


# ---------------------------------------------------------------- act-order

def test_gidx_identity_equals_plain(orc):
    p = Problem(GPTQ, M=2, K=512, N=32, G=128, seed=51)
    g = (np.arange(p.K) // p.G).astype(np.int32)
    a = orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, g_idx=g)
    b = orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_gidx_permutation_invariant(orc):
    """y(x, Q, g_idx) == y(x[:, P], Q[P], k/G) where P sorts rows by group."""
    p = Problem(GPTQ, M=3, K=512, N=32, G=128, seed=52, act_order=True)
    P = np.argsort(p.g_idx, kind="stable")
    assert np.array_equal(p.g_idx[P], np.arange(p.K) // p.G)
    y_act = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                           g_idx=p.g_idx, want_f32=True)[1]
    qw_sorted = synth.pack_gptq_qweight(p.q[P])
    y_plain = orc.w4a16_gemm(GPTQ, np.ascontiguousarray(p.x[:, P]), qw_sorted, p.scales,
                             p.qzeros, p.K, p.N, p.G, want_f32=True)[1]
    assert np.allclose(y_act, y_plain, rtol=1e-6, atol=1e-6)
    # and the group lookup really uses g_idx: ignoring it changes the result
    y_wrong = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                             want_f32=True)[1]
    assert not np.allclose(y_act, y_wrong, rtol=1e-3, atol=1e-3)


def test_gidx_out_of_range_rejected(orc):
    p = Problem(GPTQ, M=1, K=256, N=16, G=128, seed=53)
    bad = np.zeros(p.K, dtype=np.int32)
    bad[5] = 2
    with pytest.raises(ValueError):
        orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, g_idx=bad)


# ---------------------------------------------------------------- MoE

def test_moe_route_matches_numpy(orc):
    g = np.random.default_rng(61)
    logits = g.standard_normal((64, 8)).astype(np.float32)
    ids, w = orc.moe_route(logits, 2)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :2]
    assert np.array_equal(ids, top)
    pw = np.take_along_axis(p, top, 1)
    assert np.allclose(w, pw / pw.sum(1, keepdims=True), rtol=1e-6)
    # ties keep the lower expert index
    ids_t, _ = orc.moe_route(np.zeros((1, 8), dtype=np.float32), 2)
    assert ids_t.tolist() == [[0, 1]]


def test_moe_align_invariants(orc):
    g = np.random.default_rng(62)
    T, E, topk, BM = 100, 8, 2, 16
    ids, _ = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    sorted_ids, expert_ids, n = orc.moe_align(ids, E, BM)
    P = T * topk
    assert n % BM == 0 and n == sorted_ids.size and expert_ids.size == n // BM
    real = sorted_ids[sorted_ids < P]
    assert np.array_equal(np.sort(real), np.arange(P))          # every pair exactly once
    assert np.all(sorted_ids[sorted_ids >= P] == P)              # sentinel padding
    flat = ids.ravel()
    for b in range(n // BM):
        blk = sorted_ids[b * BM:(b + 1) * BM]
        blk = blk[blk < P]
        assert np.all(flat[blk] == expert_ids[b])                # block is one expert
        assert np.all(np.diff(blk) > 0)                          # stable by pair index
    assert np.all(np.diff(expert_ids) >= 0)                      # experts in order
    counts = np.bincount(flat, minlength=E)
    assert n == int(sum((c + BM - 1) // BM * BM for c in counts))


def test_moe_forward_composition(orc):
    """Fused MoE == per-pair composition of already-pinned oracle pieces."""
    g = np.random.default_rng(63)
    T, K, I, E, topk, G = 8, 128, 64, 4, 2, 64
    x = synth.rand_x(g, T, K)
    ids, w = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    w13, w2 = [], []
    for e in range(E):
        p1 = Problem(GPTQ, 1, K, 2 * I, G, seed=100 + e)
        p2 = Problem(GPTQ, 1, I, K, G, seed=200 + e)
        w13.append(orc.dequant(GPTQ, p1.qweight, p1.scales, p1.qzeros, K, 2 * I, G))
        w2.append(orc.dequant(GPTQ, p2.qweight, p2.scales, p2.qzeros, I, K, G))
    y = orc.moe_forward(x, ids, w, w13, w2)
    for t in range(T):
        acc = np.zeros(K, dtype=np.float64)
        for j in range(topk):
            e = ids[t, j]
            h = orc.gemm_f16(x[t:t + 1], w13[e], acc64=False)
            a = orc.silu_mul_f16(h[0, :I], h[0, I:]).reshape(1, I)
            ye = orc.gemm_f16(a, w2[e], acc64=False)
            acc += float(w[t, j]) * ye[0].astype(np.float64)
        assert np.array_equal(y[t].view(np.uint16),
                              acc.astype(np.float32).astype(np.float16).view(np.uint16))


def test_silu_mul_f32_closed_form_and_special_values(orc):
    """elementwise.rs:214-250 in f32: against float64 silu(g) * u within the error of three
    f32 roundings and one expf (a few ulps), exact special values, and the interleaved
    indexing (gate first, up `inter` elements on, a last row cut short) against the
    element function."""
    g = np.random.default_rng(65)
    a = (g.standard_normal(5000) * 6).astype(np.float32)
    b = (g.standard_normal(5000) * 3).astype(np.float32)
    got = np.array([orc.lib().orc_silu_mul_f32(float(x), float(y)) for x, y in zip(a, b)],
                   dtype=np.float32).astype(np.float64)
    af, bf = a.astype(np.float64), b.astype(np.float64)
    want = af / (1.0 + np.exp(-af)) * bf
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * ulp + 1e-37)
    f = lambda x, y: orc.lib().orc_silu_mul_f32(x, y)
    assert f(0.0, 5.0) == 0.0
    assert f(100.0, 3.0) == 300.0                       # exp(-100) vanishes beside 1
    assert f(-100.0, 3.0) == 0.0                        # exp(100) overflows: g / inf
    assert f(2.0, 0.0) == 0.0
    assert abs(f(1.0, 1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 2e-7
    # interleaved rows: 5 rows of inter = 7, the last row cut after 3 entries
    rows, inter = 5, 7
    gu = (g.standard_normal((rows, 2 * inter)) * 4).astype(np.float32)
    total = rows * inter - 4
    out = orc.silu_mul_f32_rows(gu, inter, total)
    elem = np.array([f(float(gu[i // inter, i % inter]), float(gu[i // inter, inter + i % inter]))
                     for i in range(total)], dtype=np.float32)
    assert np.array_equal(out.view(np.uint32), elem.view(np.uint32))
    swapped = np.array([f(float(gu[i // inter, inter + i % inter]), float(gu[i // inter, i % inter]))
                        for i in range(total)], dtype=np.float32)
    assert not np.array_equal(out, swapped)             # gate and up are not interchangeable


def test_silu_mul_error_bound(orc):
    g = np.random.default_rng(64)
    a = (g.standard_normal(4000) * 4).astype(np.float16)
    b = g.standard_normal(4000).astype(np.float16)
    got = orc.silu_mul_f16(a, b).astype(np.float64)
    af, bf = a.astype(np.float64), b.astype(np.float64)
    want = af / (1 + np.exp(-af)) * bf
    # result rounded once to fp16 from an f32 computation: within 1 fp16 ulp (+ tiny f32 slack)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp * 1.01 + 1e-7)
