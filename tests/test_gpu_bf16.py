"""GPU parity of the bfloat16 instantiation (W4A16_BF16 flag): dequantised weights bit-exact
against the oracle, GEMM outputs within the path's 1e-2 bar of the oracle's float64
accumulation and bit-exact on inputs whose every product and partial sum is exact in fp32,
on each kernel bf16 runs (VALU GEMV up to 4 rows, small-batch up to 64, pipelined prefill
beyond, AWQ's row-paired matrix-core GEMV up to 8 rows; act-order on the small-batch kernel's
group table and the group-order prefill route; the generic kernel for other shapes). The reference kernels are generic over the element
type and name bf16 (w4a16_gptq_gemm_typed.rs:65-67)."""
import numpy as np
import pytest

import synth
from helpers import assert_parity, pkg, to_dev
from synth import Problem

pytestmark = pytest.mark.gpu
GPTQ, SYM, AWQ = 0, 1, 2
FMT_NAME = {GPTQ: "gptq", SYM: "gptq_sym", AWQ: "awq"}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def bf16_bits(torch, a) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_dev(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def dev_bits(t) -> np.ndarray:
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
@pytest.mark.parametrize("transposed", [False, True])
def test_dequant_bf16_bit_exact(torch_cuda, orc, fmt, transposed):
    torch = torch_cuda
    p = Problem(fmt, M=1, K=512, N=256, G=128, seed=700 + fmt)
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    out = pkg().dequant(to_dev(p.qweight), bf16_dev(torch, s_bits),
                        None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt],
                        group_size=p.G, transposed=transposed)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    want = orc.dequant_bf16(fmt, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G, transposed=transposed)
    assert np.array_equal(dev_bits(out), want)


def test_dequant_bf16_act_order_bit_exact(torch_cuda, orc):
    torch = torch_cuda
    p = Problem(GPTQ, M=1, K=1024, N=128, G=128, seed=710, act_order=True)
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    out = pkg().dequant(to_dev(p.qweight), bf16_dev(torch, s_bits), to_dev(p.qzeros),
                        fmt="gptq", group_size=p.G, g_idx=to_dev(p.g_idx))
    torch.cuda.synchronize()
    want = orc.dequant_bf16(GPTQ, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G, g_idx=p.g_idx)
    assert np.array_equal(dev_bits(out), want)


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
@pytest.mark.parametrize("M,K,N,kernel", [(1, 1024, 512, "gemv"), (7, 512, 256, "skinny"),
                                          (64, 2048, 768, "skinny"), (200, 1024, 512, "prefill"),
                                          (33, 384, 136, "strided")])
def test_gemm_bf16_matches_oracle(torch_cuda, orc, fmt, M, K, N, kernel):
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=720 + M + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, p.G, bf16=True) == kernel
    x_bits = bf16_bits(torch, p.x.astype(np.float32))
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    y = P.gemm(bf16_dev(torch, x_bits), to_dev(p.qweight), bf16_dev(torch, s_bits),
               None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt], group_size=p.G)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    _, ref = orc.w4a16_gemm_bf16(fmt, x_bits, p.qweight, s_bits, p.qzeros, K, N, p.G)
    assert_parity(y.float().cpu().numpy(), ref, what=f"bf16 fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt,M,K,N,kernel", [
    (AWQ, 1, 4096, 14336, "gemv"),        # config 1's shapes in bf16
    (AWQ, 1, 14336, 4096, "gemv"),
    (AWQ, 4, 4096, 14336, "gemv"),
    (AWQ, 5, 4096, 14336, "gemv"),        # row-paired matrix-core GEMV
    (AWQ, 8, 14336, 4096, "gemv"),
    (GPTQ, 8, 4096, 14336, "skinny"),
    (SYM, 1, 4096, 4096, "gemv"),         # config 0's shape
    (GPTQ, 3, 14336, 4096, "gemv"),
    (GPTQ, 16, 4096, 6144, "skinny"),     # config 2's shape, plain group order
    (GPTQ, 64, 4096, 6144, "skinny"),
    (SYM, 256, 8192, 1024, "prefill"),    # prefill with its K split across workgroups
    (AWQ, 2048, 4096, 14336, "prefill"),  # config 3
])
def test_gemm_bf16_fast_paths_full_size(torch_cuda, orc, fmt, M, K, N, kernel):
    """The bf16 GEMV, small-batch and prefill kernels at the benchmark shapes: every row up to 16
    rows, else 16 sampled rows (the first and last among them), against the oracle's bf16
    GEMM; a second call is bit-identical (fixed-order split-K sums)."""
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0xBF160000 + M + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, p.G, bf16=True) == kernel
    x_bits = bf16_bits(torch, p.x.astype(np.float32))
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    args = (bf16_dev(torch, x_bits), to_dev(p.qweight), bf16_dev(torch, s_bits),
            None if p.qzeros is None else to_dev(p.qzeros))
    y = P.gemm(*args, fmt=FMT_NAME[fmt], group_size=p.G)
    y2 = P.gemm(*args, fmt=FMT_NAME[fmt], group_size=p.G)
    torch.cuda.synchronize()
    assert np.array_equal(dev_bits(y), dev_bits(y2))
    if M <= 16:
        rows = np.arange(M)
    else:
        rows = np.random.default_rng(M).choice(M, 16, replace=False)
        rows[:2] = [0, M - 1]
    _, ref = orc.w4a16_gemm_bf16(fmt, x_bits[rows], p.qweight, s_bits, p.qzeros, K, N, p.G)
    got = y.float().cpu().numpy()[rows]
    assert np.all(np.isfinite(got))
    assert_parity(got, ref, what=f"bf16 {kernel} fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt,M,K,N,kernel", [(GPTQ, 16, 1024, 256, "skinny"),
                                               (GPTQ, 16, 4096, 6144, "skinny"),   # config 2, bf16
                                               (SYM, 64, 4096, 6144, "skinny"),
                                               (GPTQ, 2048, 4096, 6144, "prefill"),
                                               (GPTQ, 33, 384, 136, "strided")])
def test_gemm_bf16_act_order_matches_oracle(torch_cuda, orc, fmt, M, K, N, kernel):
    """bf16 act-order: the small-batch kernel's group table up to 64 rows, the group-order
    prefill route beyond (per-call permutation, row repack and column gather), the generic
    kernel for shapes neither takes; every row up to 16 rows, else 16 sampled rows."""
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=730 + M + fmt, act_order=True)
    assert P.plan(FMT_NAME[fmt], M, N, K, p.G, has_g_idx=True, bf16=True) == kernel
    x_bits = bf16_bits(torch, p.x.astype(np.float32))
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    y = P.gemm(bf16_dev(torch, x_bits), to_dev(p.qweight), bf16_dev(torch, s_bits),
               None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt], group_size=p.G,
               g_idx=to_dev(p.g_idx))
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 16 else np.random.default_rng(M).choice(M, 16, replace=False)
    _, ref = orc.w4a16_gemm_bf16(fmt, x_bits[rows], p.qweight, s_bits, p.qzeros, K, N, p.G,
                                 g_idx=p.g_idx)
    assert_parity(y.float().cpu().numpy()[rows], ref, what=f"bf16 act-order {kernel} M={M}")


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
@pytest.mark.parametrize("M,G,kernel", [(1, 32, "gemv"), (1, 64, "gemv"), (1, 256, "gemv"),
                                        (4, 64, "gemv"), (6, 64, "skinny"), (16, 32, "skinny"),
                                        (200, 64, "prefill"), (200, 256, "prefill")])
def test_gemm_bf16_group_sizes(torch_cuda, orc, fmt, M, G, kernel):
    """Group sizes 32 to 256 on each bf16 kernel (K = 2048, N = 512); 16 sampled rows at
    M = 200."""
    torch = torch_cuda
    P = pkg()
    K, N = 2048, 512
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=780 + M + G + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, G, bf16=True) == kernel
    x_bits = bf16_bits(torch, p.x.astype(np.float32))
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    y = P.gemm(bf16_dev(torch, x_bits), to_dev(p.qweight), bf16_dev(torch, s_bits),
               None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt], group_size=G)
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 16 else np.random.default_rng(G).choice(M, 16, replace=False)
    _, ref = orc.w4a16_gemm_bf16(fmt, x_bits[rows], p.qweight, s_bits, p.qzeros, K, N, G)
    assert_parity(y.float().cpu().numpy()[rows], ref, what=f"bf16 {kernel} fmt={fmt} M={M} G={G}")


def test_gemm_bf16_act_order_unequal_groups_runs_generic(torch_cuda, orc):
    """Beyond 64 rows a g_idx whose groups do not each hold G rows fails the device-side
    check of the prefill route, and the gated generic kernel runs in bf16."""
    torch = torch_cuda
    p = Problem(GPTQ, M=96, K=1024, N=256, G=128, seed=1337)
    g_idx = np.random.default_rng(1337).integers(0, p.K // p.G, p.K).astype(np.int32)
    g_idx[:5] = 0
    x_bits = bf16_bits(torch, p.x.astype(np.float32))
    s_bits = bf16_bits(torch, p.scales.astype(np.float32))
    y = pkg().gemm(bf16_dev(torch, x_bits), to_dev(p.qweight), bf16_dev(torch, s_bits),
                   to_dev(p.qzeros), fmt="gptq", group_size=p.G, g_idx=to_dev(g_idx))
    torch.cuda.synchronize()
    _, ref = orc.w4a16_gemm_bf16(GPTQ, x_bits, p.qweight, s_bits, p.qzeros, p.K, p.N, p.G,
                                 g_idx=g_idx)
    assert_parity(y.float().cpu().numpy(), ref, what="bf16 act-order unequal groups")


@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
@pytest.mark.parametrize("M,K,N,G", [(9, 256, 128, 64), (1, 4096, 512, 128), (3, 4096, 1024, 128),
                                     (6, 4096, 1024, 128), (40, 4096, 768, 128), (256, 8192, 1024, 128)])
def test_gemm_bf16_exact_inputs_bit_exact(torch_cuda, orc, fmt, M, K, N, G):
    """x in multiples of 1/2 up to 2, scales 2^-7: every product and partial sum is exact in
    fp32, so the output is the exact sum rounded once to bf16, identical to the oracle, on
    the GEMVs (1 and 3 rows, and AWQ's row-paired one at 6; K split with the fixed-point
    hand-off), the small-batch kernel
    (with and without a K split across workgroups) and the prefill kernel (256 rows: K split
    in 4)."""
    torch = torch_cuda
    g = np.random.default_rng(740 + fmt)
    q = g.integers(0, 16, size=(K, N), dtype=np.int32)
    zq = g.integers(0, 16, size=(K // G, N), dtype=np.int32)
    if fmt == AWQ:
        qweight, qzeros = synth.pack_along_n(q, awq=True), synth.pack_along_n(zq, awq=True)
    else:
        qweight = synth.pack_gptq_qweight(q)
        qzeros = synth.pack_along_n(zq, awq=False) if fmt == GPTQ else None
    x = g.integers(-4, 5, size=(M, K)).astype(np.float32) / 2
    x_bits = bf16_bits(torch, x)
    s_bits = bf16_bits(torch, np.full((K // G, N), 2.0 ** -7, dtype=np.float32))
    y = pkg().gemm(bf16_dev(torch, x_bits), to_dev(qweight), bf16_dev(torch, s_bits),
                   None if qzeros is None else to_dev(qzeros), fmt=FMT_NAME[fmt], group_size=G)
    torch.cuda.synchronize()
    want, _ = orc.w4a16_gemm_bf16(fmt, x_bits, qweight, s_bits, qzeros, K, N, G)
    assert np.array_equal(dev_bits(y), want)


@pytest.mark.parametrize("fmt,M,K,N,kernel", [(AWQ, 4, 1024, 512, "gemv"),
                                               (GPTQ, 16, 4096, 6144, "skinny"),
                                               (SYM, 128, 8192, 1024, "prefill")])
def test_noalloc_bf16_equals_gemm(torch_cuda, fmt, M, K, N, kernel):
    """The allocation-free entry in bf16 runs the same kernels, with their K splits in its
    fixed scratch area (the prefill case: 256 x 128 tiles in 8 splits, 4.2 MB of partials):
    bit-identical outputs."""
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=750 + M)
    assert P.plan(FMT_NAME[fmt], M, N, K, 128, bf16=True) == kernel
    x = bf16_dev(torch, bf16_bits(torch, p.x.astype(np.float32)))
    s = bf16_dev(torch, bf16_bits(torch, p.scales.astype(np.float32)))
    qw = to_dev(p.qweight)
    qz = None if p.qzeros is None else to_dev(p.qzeros)
    y = P.gemm(x, qw, s, qz, fmt=FMT_NAME[fmt])
    out = torch.empty_like(y)
    P.gemm_noalloc(x, qw, s, qz, out, fmt=FMT_NAME[fmt])
    torch.cuda.synchronize()
    assert np.array_equal(dev_bits(out), dev_bits(y))


def test_bf16_element_types_must_agree(torch_cuda):
    torch = torch_cuda
    P = pkg()
    p = Problem(AWQ, M=2, K=256, N=256, G=128, seed=760)
    x = to_dev(p.x).to(torch.bfloat16)
    with pytest.raises(P.InvalidArgument, match="scales has dtype"):
        P.gemm(x, to_dev(p.qweight), to_dev(p.scales), to_dev(p.qzeros), fmt="awq")
    with pytest.raises(P.InvalidArgument, match="out"):
        P.gemm(x, to_dev(p.qweight), to_dev(p.scales).to(torch.bfloat16), to_dev(p.qzeros),
               fmt="awq", out=torch.empty((2, 256), dtype=torch.float16, device="cuda:0"))
