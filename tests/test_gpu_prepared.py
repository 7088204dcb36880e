"""Prepared (kernel-native) layout: the one-time repack (w4a16_prepare_layout) against an
independent numpy restatement of the layout, the dequantisation of prepared weights bit for
bit against the oracle's dequantisation of the checkpoint, and the GEMM on prepared weights
against the oracle's GEMM on the checkpoint (crates/triton-dsl/examples/
w4a16_gptq_gemm_typed.rs:130-273, awq_gemm_int4_typed.rs:116-241), for all three formats,
act-order through the group-order repack included."""
import numpy as np
import pytest

from helpers import assert_parity, pkg, to_dev
from synth import Problem, prepared_layout

pytestmark = pytest.mark.gpu
GPTQ, SYM, AWQ = 0, 1, 2
NAME = {GPTQ: "gptq", SYM: "gptq_sym", AWQ: "awq"}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _prep(P, p, zo=None):
    zo = p.zero_offset if zo is None else zo
    return P.prepare_layout(to_dev(p.qweight), to_dev(p.scales),
                            None if p.qzeros is None else to_dev(p.qzeros), fmt=NAME[p.fmt],
                            group_size=p.G, zero_offset=zo)


@pytest.mark.parametrize("fmt,K,N,G,zo", [
    (AWQ, 256, 64, 128, 0), (GPTQ, 512, 96, 64, 1), (SYM, 384, 48, 32, 0), (GPTQ, 1024, 32, 256, 0),
    (AWQ, 4096, 128, 4096, 0), (AWQ, 1536, 32, 512, 0),
])
def test_prepare_layout_bytes(torch_cuda, fmt, K, N, G, zo):
    P = pkg()
    p = Problem(fmt, M=1, K=K, N=N, G=G, seed=7000 + K + N, zero_offset=zo)
    w = _prep(P, p)
    torch_cuda.cuda.synchronize()
    assert w.buffer.numel() == P.prepared_bytes(K, N, G)
    want = prepared_layout(p.q, p.zero_int(), p.scales, G)
    assert np.array_equal(w.buffer.cpu().numpy(), want)


@pytest.mark.parametrize("fmt,K,N,G", [(AWQ, 1024, 256, 128), (GPTQ, 512, 160, 32), (SYM, 768, 64, 64)])
@pytest.mark.parametrize("transposed", [False, True])
def test_dequant_prepared_bit_exact(torch_cuda, orc, fmt, K, N, G, transposed):
    P = pkg()
    p = Problem(fmt, M=1, K=K, N=N, G=G, seed=7100 + K)
    w16 = P.dequant_prepared(_prep(P, p), transposed=transposed).cpu().numpy()
    ref = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, K, N, G, zero_offset=p.zero_offset)
    if transposed:
        ref = ref.T
    assert np.array_equal(w16.view(np.uint16), np.ascontiguousarray(ref).view(np.uint16))


@pytest.mark.parametrize("fmt,M,K,N,G", [
    (AWQ, 1, 4096, 14336, 128),     # config 1 (M = 1), both MLP shapes
    (AWQ, 1, 14336, 4096, 128),
    (SYM, 1, 4096, 4096, 128),      # config 0
    (GPTQ, 1, 4096, 6144, 128),
    (AWQ, 1, 1024, 512, 32), (GPTQ, 1, 2048, 1792, 64), (SYM, 1, 384, 80, 128),
    (AWQ, 1, 1792, 4096, 128), (AWQ, 1, 4096, 1792, 128),   # one GPU's share of an 8-way TP MLP
    (GPTQ, 1, 32768, 256, 128), (AWQ, 1, 128, 16, 128), (AWQ, 1, 4096, 512, 256),
    (GPTQ, 1, 2048, 256, 2048), (SYM, 1, 4096, 1024, 32),
    # M = 2..8: config 1's shapes at M = 4 and 8, every M on a smaller shape
    (AWQ, 4, 4096, 14336, 128), (AWQ, 8, 4096, 14336, 128), (AWQ, 4, 14336, 4096, 128),
    (AWQ, 8, 14336, 4096, 128), (GPTQ, 2, 1024, 512, 128), (GPTQ, 3, 1024, 512, 128),
    (SYM, 5, 2048, 256, 128), (AWQ, 6, 1536, 64, 256), (GPTQ, 7, 512, 32, 128),
    (AWQ, 2, 128, 16, 128), (AWQ, 8, 16384, 128, 128),
    # 3..4 rows, two strips per workgroup: an odd strip count, 16 waves of 4 blocks
    (SYM, 4, 1024, 16 * 33, 128), (AWQ, 3, 8192, 272, 128),
])
def test_gemm_prepared_matches_oracle(torch_cuda, orc, fmt, M, K, N, G):
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=0x5EED0001 + K + N)
    w = _prep(P, p)
    y = P.gemm_prepared(to_dev(p.x), w)
    y2 = P.gemm_prepared(to_dev(p.x), w)
    torch_cuda.cuda.synchronize()
    y, y2 = y.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16)), "repeated calls differ"
    ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G,
                         zero_offset=p.zero_offset, want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"prepared {NAME[fmt]} M={M} K={K} N={N} G={G}")


def test_gemm_prepared_exact_arithmetic(torch_cuda, orc):
    """x = j/4 and power-of-two scales: every product and partial sum is exact in fp32, so the
    output is the exact sum rounded once to fp16 — bit for bit the oracle's."""
    P = pkg()
    g = np.random.default_rng(77)
    for fmt in (AWQ, GPTQ, SYM):
        p = Problem(fmt, M=1, K=2048, N=512, G=128, seed=78 + fmt)
        p.x = (g.integers(-8, 9, size=p.x.shape) / 4.0).astype(np.float16)
        p.scales = (2.0 ** g.integers(-8, -4, size=p.scales.shape)).astype(np.float16)
        y = P.gemm_prepared(to_dev(p.x), _prep(P, p)).cpu().numpy()
        ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                             zero_offset=p.zero_offset)
        assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)), NAME[fmt]


@pytest.mark.parametrize("M,K,N", [(1, 4096, 6144), (1, 1024, 384)])
def test_act_order_then_prepared(torch_cuda, orc, M, K, N):
    """An act-order checkpoint: group-order repack, then the prepared layout of the repacked
    weights; the product with x gathered by perm equals the act-order GEMM."""
    P = pkg()
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED0002 + K, act_order=True)
    qout, perm = P.prepare_act_order(to_dev(p.qweight), to_dev(p.g_idx), group_size=128)
    w = P.prepare_layout(qout, to_dev(p.scales), to_dev(p.qzeros), fmt="gptq", group_size=128,
                         zero_offset=1)
    w16 = P.dequant_prepared(w).cpu().numpy()
    ref_w = orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, K, N, 128, g_idx=p.g_idx)
    perm_h = perm.cpu().numpy()
    assert np.array_equal(w16.view(np.uint16), ref_w[perm_h].view(np.uint16))
    y = P.gemm_prepared(to_dev(p.x), w, perm=perm).cpu().numpy()
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, g_idx=p.g_idx,
                         want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what="act-order prepared")


@pytest.mark.parametrize("fmt,M,K,N,G", [
    (AWQ, 9, 1024, 512, 128), (GPTQ, 16, 2048, 768, 128), (AWQ, 64, 4096, 1024, 64),
    (SYM, 100, 1024, 256, 256), (GPTQ, 300, 2048, 4096, 128),    # prefill tiles, K split
    (AWQ, 130, 1024, 224, 128),                                  # 224-column tiles
    (AWQ, 128, 14336, 4096, 128),                                # K split in 8
    (GPTQ, 40, 512, 48, 32), (AWQ, 12, 16384 + 128, 32, 128),    # generic kernel (G = 32, K)
])
def test_gemm_prepared_large_m_matches_oracle(torch_cuda, orc, fmt, M, K, N, G):
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=0x5EED0003 + M + K + N)
    y = P.gemm_prepared(to_dev(p.x), _prep(P, p)).cpu().numpy()
    rows = np.arange(M) if M <= 64 else np.unique(np.r_[0, M - 1, np.random.default_rng(M).choice(M, 30)])
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G,
                              rows.astype(np.int32), zero_offset=p.zero_offset)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prepared {NAME[fmt]} M={M} K={K} N={N} G={G}")


@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
def test_gemm_prepared_config3_sampled_rows(torch_cuda, orc, K, N):
    """Config 3 (AWQ, M = 2048) through the prepared layout; 32 sampled rows against the
    oracle, and bit-identical to the checkpoint kernel on exactly representable inputs is not
    required (different accumulation order), so the bar is the tolerance."""
    P = pkg()
    M = 2048
    p = Problem(AWQ, M=M, K=K, N=N, G=128, seed=0x5EED0003 + K)
    y = P.gemm_prepared(to_dev(p.x), _prep(P, p)).cpu().numpy()
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(K).choice(M, 30)]).astype(np.int32)
    ref = orc.w4a16_gemm_rows(AWQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows, zero_offset=0)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prepared config 3 K={K} N={N}")


def test_gemm_prepared_prefill_exact_arithmetic(torch_cuda, orc):
    """Exactly representable products and sums: the prefill and generic kernels on prepared
    weights give the oracle's bits."""
    P = pkg()
    g = np.random.default_rng(79)
    for fmt, M, K, N, G in ((AWQ, 96, 1024, 256, 128), (GPTQ, 20, 512, 48, 32), (SYM, 70, 2048, 512, 64)):
        p = Problem(fmt, M=M, K=K, N=N, G=G, seed=80 + fmt)
        p.x = (g.integers(-8, 9, size=p.x.shape) / 4.0).astype(np.float16)
        p.scales = (2.0 ** g.integers(-8, -4, size=p.scales.shape)).astype(np.float16)
        y = P.gemm_prepared(to_dev(p.x), _prep(P, p)).cpu().numpy()
        ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                             zero_offset=p.zero_offset)
        assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)), (NAME[fmt], M)


# ------------------------------------------------- small batch (5..64 rows, G % 128 == 0)

@pytest.mark.parametrize("fmt,M,K,N,G", [
    (GPTQ, 16, 4096, 6144, 128), (GPTQ, 32, 4096, 6144, 128), (GPTQ, 64, 4096, 6144, 128),  # config 2's shape
    (AWQ, 8, 4096, 14336, 128), (AWQ, 8, 14336, 4096, 128),      # config 1 at M = 8: 4 and 1 strips per workgroup
    (AWQ, 17, 4096, 16 * 385, 128),     # 2 strips per workgroup, the last one holds one
    (SYM, 33, 1024, 16 * 771, 128),     # 4 strips per workgroup (3 in the last), 3 row tiles
    (GPTQ, 47, 128 * 33, 512, 128),     # 8 blocks per wave, the last wave 1 block
    (AWQ, 63, 128 * 70, 256, 256),      # 16 blocks per wave, group of 2 blocks
    (GPTQ, 5, 32768, 64, 128),          # 32 blocks per wave, 8 waves
    (SYM, 12, 128, 16, 128),            # one block, one strip
    # x streamed through the waves' LDS slots: 2 row tiles with 8 blocks per wave; one tile
    # with a last wave of 5 blocks (3 past K); all of x up front with a last wave of 1 block;
    # 4 rows (the rows GEMV's range) where a wave takes 4 blocks
    (GPTQ, 24, 8192, 512, 128), (AWQ, 9, 128 * 37, 128, 128), (SYM, 10, 128 * 13, 96, 128),
    (GPTQ, 4, 2048, 320, 128),
])
def test_gemm_prepared_small_batch_matches_oracle(torch_cuda, orc, fmt, M, K, N, G):
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=0x5EED0005 + M + K + N)
    w = _prep(P, p)
    y = P.gemm_prepared(to_dev(p.x), w)
    y2 = P.gemm_prepared(to_dev(p.x), w)
    torch_cuda.cuda.synchronize()
    y, y2 = y.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16)), "repeated calls differ"
    ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G,
                         zero_offset=p.zero_offset, want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"prepared small batch {NAME[fmt]} M={M} K={K} N={N} G={G}")


@pytest.mark.parametrize("M", [2, 7, 16, 32, 64])
def test_act_order_then_prepared_small_batch(torch_cuda, orc, M):
    """Config 2 (GPTQ act-order, K=4096 -> N=6144) through the group-order repack and the
    prepared layout: x's columns are gathered by the permutation, then the small-batch kernel
    reads the gathered rows (with a permutation it serves every M from 2)."""
    P = pkg()
    K, N = 4096, 6144
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED0002 + M, act_order=True)
    qout, perm = P.prepare_act_order(to_dev(p.qweight), to_dev(p.g_idx), group_size=128)
    w = P.prepare_layout(qout, to_dev(p.scales), to_dev(p.qzeros), fmt="gptq", group_size=128,
                         zero_offset=1)
    y = P.gemm_prepared(to_dev(p.x), w, perm=perm).cpu().numpy()
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, g_idx=p.g_idx,
                         want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"act-order prepared M={M}")


@pytest.mark.parametrize("M,K,N", [(5, 1152, 192), (16, 2048, 6160), (11, 4096, 512)])
def test_act_order_then_prepared_uneven_shapes(torch_cuda, orc, M, K, N):
    """The group-order repack, the prepared layout and the per-call gather at shapes the
    config-2 cases miss: K = 1152 leaves the small-batch kernel's last wave one block of four,
    N = 6160 an odd strip count; against the oracle's act-order GEMM on the checkpoint."""
    P = pkg()
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED0330 + M + K, act_order=True)
    qout, perm = P.prepare_act_order(to_dev(p.qweight), to_dev(p.g_idx), group_size=128)
    w = P.prepare_layout(qout, to_dev(p.scales), to_dev(p.qzeros), fmt="gptq", group_size=128,
                         zero_offset=1)
    y = P.gemm_prepared(to_dev(p.x), w, perm=perm).cpu().numpy()
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, g_idx=p.g_idx,
                         want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"act-order prepared M={M} K={K} N={N}")


def test_gemm_prepared_small_batch_exact_arithmetic(torch_cuda, orc):
    """Exactly representable products and sums through the small-batch kernel (every row-tile
    count, with and without act-order): the oracle's bits."""
    P = pkg()
    g = np.random.default_rng(81)
    for fmt, M, K, N, G, act in ((AWQ, 16, 1024, 512, 128, False), (GPTQ, 29, 2048, 256, 256, False),
                                 (SYM, 48, 512, 6160, 128, False), (GPTQ, 64, 2048, 192, 128, True),
                                 (GPTQ, 3, 1024, 64, 128, True)):
        p = Problem(fmt, M=M, K=K, N=N, G=G, seed=82 + M, act_order=act)
        p.x = (g.integers(-8, 9, size=p.x.shape) / 4.0).astype(np.float16)
        p.scales = (2.0 ** g.integers(-8, -4, size=p.scales.shape)).astype(np.float16)
        if act:
            qout, perm = P.prepare_act_order(to_dev(p.qweight), to_dev(p.g_idx), group_size=G)
            w = P.prepare_layout(qout, to_dev(p.scales), to_dev(p.qzeros), fmt="gptq", group_size=G,
                                 zero_offset=p.zero_offset)
            y = P.gemm_prepared(to_dev(p.x), w, perm=perm).cpu().numpy()
        else:
            y = P.gemm_prepared(to_dev(p.x), _prep(P, p)).cpu().numpy()
        ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                             g_idx=p.g_idx if act else None, zero_offset=p.zero_offset)
        assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)), (NAME[fmt], M, act)


@pytest.mark.parametrize("fmt,M,K,N,G", [
    (GPTQ, 16, 4096, 6144, 128), (GPTQ, 64, 4096, 6144, 128),   # config 2, as stored + g_idx
    (GPTQ, 1, 2048, 512, 128), (GPTQ, 7, 1024, 6160, 128), (SYM, 40, 2048, 1024, 128),
    (GPTQ, 24, 1024, 512, 32), (SYM, 9, 512, 2048, 64), (GPTQ, 33, 4096, 256, 256),
    (GPTQ, 16, 4096, 6144, 32), (GPTQ, 48, 4096, 6144, 32),    # the largest table: 4096 entries
    (GPTQ, 100, 1024, 256, 128), (GPTQ, 5, 8192, 128, 128),     # generic kernel: M > 64, K > 4096
])
def test_gemm_prepared_gidx_matches_oracle(torch_cuda, orc, fmt, M, K, N, G):
    """An act-order checkpoint prepared as stored (rows in their own order) with g_idx
    (w4a16_gemm_prepared_gidx): the small-batch kernel's (scale, zero) table filled from the
    strips' tables, or the generic kernel reading each group's table row; against the oracle's
    act-order GEMM on the checkpoint."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=0x5EED0300 + M + K, act_order=True)
    y = P.gemm_prepared(to_dev(p.x), _prep(P, p), g_idx=to_dev(p.g_idx)).cpu().numpy()
    ref = orc.w4a16_gemm(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G, g_idx=p.g_idx,
                         zero_offset=p.zero_offset, want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"prepared g_idx {NAME[fmt]} M={M} K={K} N={N} G={G}")


@pytest.mark.parametrize("fmt,M,G", [(GPTQ, 32, 128), (GPTQ, 64, 128), (SYM, 48, 128), (GPTQ, 40, 64)])
def test_gemm_prepared_gidx_equals_checkpoint_route(torch_cuda, fmt, M, G):
    """Beyond 16 rows w4a16_gemm runs the same small-batch kernel on the checkpoint as stored
    (K = 4096 over 8 waves of 4 blocks, the same W16 per weight and the same MFMA chain): on
    the prepared strips with g_idx the output is bit for bit the checkpoint call's."""
    P = pkg()
    K, N = 4096, 6144
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=0x5EED0310 + M, act_order=True)
    g_idx = to_dev(p.g_idx)
    y = P.gemm_prepared(to_dev(p.x), _prep(P, p), g_idx=g_idx).cpu().numpy()
    assert P.plan(NAME[fmt], M, N, K, G, has_g_idx=True) == "skinny"
    ck = P.gemm(to_dev(p.x), to_dev(p.qweight), to_dev(p.scales),
                None if p.qzeros is None else to_dev(p.qzeros), fmt=NAME[fmt], group_size=G,
                g_idx=g_idx, zero_offset=p.zero_offset).cpu().numpy()
    assert np.array_equal(y.view(np.uint16), ck.view(np.uint16))


def test_gemm_prepared_gidx_clamps_and_unequal_groups(torch_cuda, orc):
    """g_idx entries outside [0, K/G) are clamped into the table (as w4a16_gemm does), and
    groups of unequal size need nothing else: each row reads its own group's entry."""
    P = pkg()
    p = Problem(GPTQ, M=20, K=1024, N=512, G=128, seed=0x5EED0320, act_order=True)
    bad = p.g_idx.copy()
    bad[3], bad[700], bad[10] = 99, -5, bad[11]
    y = P.gemm_prepared(to_dev(p.x), _prep(P, p), g_idx=to_dev(bad)).cpu().numpy()
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                         g_idx=np.clip(bad, 0, p.K // p.G - 1).astype(np.int32), want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what="prepared g_idx clamped / unequal")
