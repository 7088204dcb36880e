"""GPTQ act-order in group order: the one-time repack (w4a16_prepare_act_order) and the
gather-then-plain-kernel product (w4a16_gemm_act_order), against the oracle's act-order
GEMM on the original checkpoint (g_idx applied row by row)."""
import numpy as np
import pytest

from helpers import assert_parity, pkg, to_dev
from synth import Problem

pytestmark = pytest.mark.gpu
GPTQ, SYM = 0, 1
FMT_NAME = {GPTQ: "gptq", SYM: "gptq_sym"}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _prepare(P, p):
    return P.prepare_act_order(to_dev(p.qweight), to_dev(p.g_idx), group_size=p.G,
                               fmt=FMT_NAME[p.fmt])


@pytest.mark.parametrize("fmt,G", [(GPTQ, 128), (SYM, 64), (GPTQ, 32)])
def test_prepare_is_the_stable_group_sort_and_bit_exact(torch_cuda, orc, fmt, G):
    """perm = argsort(g_idx, stable); the repacked matrix dequantises (plain group order) to
    exactly the original's act-order dequantisation, rows permuted by perm."""
    P = pkg()
    p = Problem(fmt, M=1, K=1024, N=384, G=G, seed=6100 + G, act_order=True)
    qout, perm = _prepare(P, p)
    torch_cuda.cuda.synchronize()
    perm_h = perm.cpu().numpy()
    assert np.array_equal(perm_h, np.argsort(p.g_idx, kind="stable"))
    w_new = P.dequant(qout, to_dev(p.scales), None if p.qzeros is None else to_dev(p.qzeros),
                      fmt=FMT_NAME[fmt], group_size=G).cpu().numpy()
    w_ref = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, p.K, p.N, G, g_idx=p.g_idx)
    assert np.array_equal(w_new.view(np.uint16), w_ref[perm_h].view(np.uint16))


@pytest.mark.parametrize("fmt,M,K,N,zo", [
    (GPTQ, 1, 4096, 6144, 1),       # decode GEMV after the gather
    (GPTQ, 16, 4096, 6144, 1),      # config 2 sizes
    (GPTQ, 64, 4096, 6144, 1),
    (SYM, 8, 2048, 1024, 1),
    (GPTQ, 100, 1024, 768, 0),      # prefill (the case the g_idx kernels cannot take)
    (GPTQ, 512, 2048, 4096, 1),     # prefill with K split
])
def test_gemm_act_order_matches_oracle(torch_cuda, orc, fmt, M, K, N, zo):
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED0002 + M + K, act_order=True, zero_offset=zo)
    qout, perm = _prepare(P, p)
    y = P.gemm_act_order(to_dev(p.x), qout, to_dev(p.scales),
                         None if p.qzeros is None else to_dev(p.qzeros), perm, fmt=FMT_NAME[fmt],
                         group_size=p.G, zero_offset=zo)
    torch_cuda.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.arange(M) if M <= 64 else np.unique(np.r_[0, M - 1,
                                                        np.random.default_rng(M).choice(M, 14)])
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, p.G,
                              rows.astype(np.int32), g_idx=p.g_idx, zero_offset=zo)
    assert_parity(y[rows], ref.astype(np.float64), what=f"act-order prepared fmt={fmt} M={M}")


def test_act_order_config2_prefill_m2048_sampled_rows(torch_cuda, orc):
    """Config 2's layer (K=4096 -> N=6144, act-order) at prefill size M=2048 through the
    prepared path; the oracle checks 16 sampled rows."""
    P = pkg()
    M, K, N = 2048, 4096, 6144
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED0002, act_order=True)
    assert P.plan("gptq", M, N, K, 128) == "prefill"
    qout, perm = _prepare(P, p)
    y = P.gemm_act_order(to_dev(p.x), qout, to_dev(p.scales), to_dev(p.qzeros), perm).cpu().numpy()
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(11).choice(M, 14)]).astype(np.int32)
    ref = orc.w4a16_gemm_rows(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows,
                              g_idx=p.g_idx)
    assert_parity(y[rows], ref.astype(np.float64), what="act-order M=2048")
    assert np.all(np.isfinite(y))


def test_prepare_rejects_uneven_groups(torch_cuda):
    P = pkg()
    p = Problem(GPTQ, M=1, K=512, N=128, G=128, seed=6200, act_order=True)
    bad = p.g_idx.copy()
    bad[np.nonzero(bad == 0)[0][0]] = 1          # group 0 loses a row, group 1 gains one
    with pytest.raises(P.InvalidArgument, match="exactly group_size"):
        P.prepare_act_order(to_dev(p.qweight), to_dev(bad), group_size=128)
    bad = p.g_idx.copy()
    bad[5] = 4
    with pytest.raises(P.InvalidArgument, match="outside"):
        P.prepare_act_order(to_dev(p.qweight), to_dev(bad), group_size=128)


@pytest.mark.parametrize("M,K", [(3, 1664), (5, 1152), (1, 4224)])
def test_gather_uneven_share(torch_cuda, orc, M, K):
    """A few rows and a K whose 8-column chunks do not divide evenly over the workgroups that
    share a row (M=3, K=1664: 208 chunks, 6 workgroups of 35, the last one 33): every output
    column still gathered once, product against the oracle's act-order GEMM."""
    P = pkg()
    p = Problem(GPTQ, M=M, K=K, N=256, G=128, seed=0x5EED4000 + K, act_order=True)
    qout, perm = _prepare(P, p)
    y = P.gemm_act_order(to_dev(p.x), qout, to_dev(p.scales), to_dev(p.qzeros), perm).cpu().numpy()
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, 256, 128, g_idx=p.g_idx,
                         want_f32=True)[1]
    assert_parity(y, ref.astype(np.float64), what=f"act-order gather M={M} K={K}")


def test_gather_fallback_kernel_with_unaligned_perm(torch_cuda, orc):
    """perm at a 4-byte (not 16-byte) offset: the gather reads x's columns straight from global
    memory (the kernel kept for unaligned buffers); same product as the staged gather."""
    torch = torch_cuda
    P = pkg()
    M, K, N = 7, 2048, 384
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED4100, act_order=True)
    qout, perm = _prepare(P, p)
    buf = torch.empty(K + 1, dtype=torch.int32, device="cuda:0")
    buf[1:] = perm
    perm_u = buf[1:]
    assert perm_u.data_ptr() % 16 != 0
    y_u = P.gemm_act_order(to_dev(p.x), qout, to_dev(p.scales), to_dev(p.qzeros), perm_u).cpu().numpy()
    y = P.gemm_act_order(to_dev(p.x), qout, to_dev(p.scales), to_dev(p.qzeros), perm).cpu().numpy()
    assert np.array_equal(y_u.view(np.uint16), y.view(np.uint16))
    ref = orc.w4a16_gemm(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, g_idx=p.g_idx,
                         want_f32=True)[1]
    assert_parity(y_u, ref.astype(np.float64), what="act-order fallback gather")
