"""GPU parity: the HIP W4A16 kernels, called through the C ABI, against the CPU oracle.

Bar: dequantised weights bit-exact; GEMM outputs within max
relative error 1e-2 (helpers.rel_err: |y - ref| / max(|ref|, rms(ref))) of the oracle's
float64-accumulated dequant-then-matmul on identical seeded inputs.
"""
import ctypes

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


def _run_gemm(torch, p: Problem, g_idx=None):
    P = pkg()
    y = P.gemm(to_dev(p.x), to_dev(p.qweight), to_dev(p.scales),
               None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[p.fmt],
               group_size=p.G, g_idx=None if g_idx is None else to_dev(g_idx),
               zero_offset=p.zero_offset)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _oracle(orc, p: Problem, g_idx=None):
    return orc.w4a16_gemm(p.fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                          g_idx=g_idx, zero_offset=p.zero_offset, want_f32=True)[1]


# ------------------------------------------------------------------ decode GEMV

@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_small(torch_cuda, orc, fmt, M):
    p = Problem(fmt, M=M, K=1024, N=512, G=128, seed=1000 + 10 * fmt + M)
    assert pkg().plan(FMT_NAME[fmt], M, p.N, p.K, p.G) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"gemv fmt={fmt} M={M}")


@pytest.mark.parametrize("M", [3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("K,N,G", [(1024, 256, 128), (3072, 768, 256), (2048, 1280, 1024),
                                   (2048, 8192, 128)])
def test_gemv_awq_row_paired(torch_cuda, orc, M, K, N, G):
    """AWQ at M = 3..8 on the row-paired matrix-core kernel (K a multiple of 1024, groups of
    128 rows or more, N a multiple of 256), all with the fixed-point hand-off (M * N within its
    73728 entries; the counter protocol of larger outputs is covered by
    test_gemv_split_k_counter_protocol). The first three shapes leave under 64 workgroups of
    8 waves, so they take 4-wave, 512-row workgroups (2, 6 and 4 splits; G=1024 spans two
    workgroups); 2048 x 8192 fills 64 workgroups of 8 waves."""
    p = Problem(AWQ, M=M, K=K, N=N, G=G, seed=5100 + 10 * M + K // 1024)
    assert pkg().plan("awq", M, N, K, G) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"awq rows M={M} K={K} N={N} G={G}")
    # repeated calls are bit-identical (split order fixed; hand-off state left clean)
    assert np.array_equal(_run_gemm(torch_cuda, p).view(np.uint16), y.view(np.uint16))


@pytest.mark.parametrize("fmt", [GPTQ, SYM])
@pytest.mark.parametrize("M,K,N", [(2, 1024, 192), (4, 2048, 320), (3, 768, 256), (2, 256, 128)])
def test_gemv_gptq_tile_widths(torch_cuda, orc, fmt, M, K, N):
    """GPTQ decode at M = 2..4: the 64-column tile where N % 64 == 0 and K % 512 == 0 (N=192,
    320 only fit it), the 128-column, 256-row tile otherwise (K=768, K=256)."""
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=1200 + 10 * fmt + M + K // 64)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, 128) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"gptq gemv fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [5, 6, 7, 8])
@pytest.mark.parametrize("K,N,G", [(1024, 512, 128), (2048, 768, 64), (512, 256, 256)])
def test_gemv_awq_matrix_core(torch_cuda, orc, M, K, N, G):
    """AWQ decode for 5 <= M <= 8: dot products on the matrix cores (block-diagonal x)."""
    p = Problem(AWQ, M=M, K=K, N=N, G=G, seed=1050 + M + K // 64)
    assert pkg().plan("awq", M, N, K, G) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"awq gemv M={M} K={K} N={N} G={G}")


@pytest.mark.parametrize("fmt,G", [(AWQ, 32), (AWQ, 64), (GPTQ, 32), (GPTQ, 64), (GPTQ, 256)])
def test_gemv_group_sizes(torch_cuda, orc, fmt, G):
    p = Problem(fmt, M=1, K=2048, N=256, G=G, seed=1100 + G)
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"gemv fmt={fmt} G={G}")


@pytest.mark.parametrize("fmt,M,K,N", [
    (SYM, 1, 4096, 4096),          # config 0: GPTQ symmetric GEMV
    (AWQ, 1, 4096, 14336),         # config 1: gate/up
    (AWQ, 1, 14336, 4096),         # config 1: down
    (AWQ, 4, 4096, 14336),
    (AWQ, 4, 14336, 4096),         # config 1, M=4, down (its own grid: 16 tiles x 14 splits)
])
def test_gemv_full_size(torch_cuda, orc, fmt, M, K, N):
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED0000 + (0 if fmt == SYM else 1))
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"full fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("fmt,M,kernel", [(AWQ, 1, "gemv"), (AWQ, 2, "gemv"), (AWQ, 3, "gemv"),
                                          (AWQ, 8, "gemv"), (GPTQ, 1, "gemv"), (GPTQ, 4, "gemv"),
                                          (SYM, 2, "gemv"), (GPTQ, 16, "skinny")])
def test_spike_inputs_give_weight_rows(torch_cuda, fmt, M, kernel, bf16):
    """x = e_k (one 1 per row, at a different k in each row) returns row k of the dequantised
    weights exactly: (bias + q) - bias - z is exact, so every output is RNE((q - z) * s) with
    nothing else added. The spikes sit at every element of a 16-byte x chunk and at block and
    group edges, so a kernel that reads a wrong element of its x fragment, or sums x over the
    wrong rows for its zero-point correction, fails here (the sum of a random x can hide it)."""
    torch = torch_cuda
    P = pkg()
    K, N, G = 1024, 512, 128
    dt = torch.bfloat16 if bf16 else torch.float16
    p = Problem(fmt, M=1, K=K, N=N, G=G, seed=0x5B1CE + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, G, bf16=bf16) == kernel
    qw = to_dev(p.qweight)
    qz = None if p.qzeros is None else to_dev(p.qzeros)
    sc = to_dev(p.scales).to(dt)
    W = P.dequant(qw, sc, qz, fmt=FMT_NAME[fmt], K=K, group_size=G)
    ks = [0, 1, 2, 3, 4, 5, 6, 7, 8, 15, 16, 31, 32, 100, 127, 128, 129, 255, 511, 513, K - 1]
    for i in range(0, len(ks), M):
        rows = (ks[i:i + M] + [0] * M)[:M]
        x = torch.zeros((M, K), dtype=dt, device="cuda:0")
        for m, k in enumerate(rows):
            x[m, k] = 1
        y = P.gemm(x, qw, sc, qz, fmt=FMT_NAME[fmt], group_size=G)
        for m, k in enumerate(rows):
            assert torch.equal(y[m], W[k]), (fmt, M, bf16, k)


def test_gemv_deterministic_and_reusable(torch_cuda, orc):
    """Split-K fix-up sums in a fixed order and leaves the workspace ready for the next call."""
    P = pkg()
    p = Problem(AWQ, M=1, K=4096, N=2048, G=128, seed=7)
    args = [to_dev(a) for a in (p.x, p.qweight, p.scales, p.qzeros)]
    ys = [P.gemm(*args, fmt="awq").cpu().numpy() for _ in range(3)]
    assert all(np.array_equal(ys[0].view(np.uint16), y.view(np.uint16)) for y in ys[1:])
    # a different shape in between, then the first again
    q = Problem(AWQ, M=2, K=1024, N=512, G=128, seed=8)
    assert_parity(_run_gemm(torch_cuda, q), _oracle(orc, q))
    y2 = P.gemm(*args, fmt="awq").cpu().numpy()
    assert np.array_equal(ys[0].view(np.uint16), y2.view(np.uint16))
    assert_parity(ys[0], _oracle(orc, p))


@pytest.mark.parametrize("fmt,M,K,N,hi,lo",
                         [(AWQ, 1, 2048, 16384, 16, -8), (GPTQ, 1, 2048, 16384, 16, -8),
                          (SYM, 1, 2048, 16384, 16, -8), (GPTQ, 3, 2048, 2048, 16, -8),
                          (SYM, 4, 2048, 2048, 16, -8), (AWQ, 2, 2048, 2048, 16, -8),
                          (AWQ, 4, 2048, 2048, 16, -8), (AWQ, 8, 2048, 2048, 16, -8),
                          (AWQ, 1, 2048, 4096, 32, -24), (GPTQ, 1, 2048, 4096, 32, -24),
                          (SYM, 1, 2048, 4096, 32, -24)])
def test_gemv_split_k_out_of_range_partials(torch_cuda, orc, fmt, M, K, N, hi, lo):
    """Split-K partials of magnitude >= 2^15 leave the fixed-point hand-off for its fp32
    path (partial stored, split bit set, added in split order by the last arrival).

    Exact arithmetic, so the output must equal the oracle bit for bit: x[m, k] is hi * 2^-m
    on the first half of K and lo * 2^-m on the second, every scale is 0.5 and q and the
    zero point are constant down each column, so every product, partial sum and output is
    a small multiple of a power of two. With hi = 16, each split covers 512 rows (VALU
    kernels, and the row-paired AWQ kernel's 4-wave tiles at M = 4, 8: partial 4096 c for
    row 0 in the first half, c = q - z, so >= 2^15 exactly when |c| >= 8; two such splits per
    entry) or 1024 rows (AWQ column-interleaved matrix-core kernel at M = 2: 8192 c,
    |c| >= 4): entries of both kinds in every call; at M = 1, N = 16384 keeps the 512-row
    tiles. K=2048, N=4096 at M = 1 leaves grids small enough for the 256-row tiles
    (8 splits): hi = 32 gives first-half partials of 4096 c (|c| >= 8) and lo = -24
    second-half partials of -3072 c (|c| >= 11), with outputs 4096 c inside the fp16 range."""
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=4242 + 10 * fmt + M + N)
    g = np.random.default_rng(4243 + 10 * fmt + M + N)
    col_q = g.integers(0, 16, size=N)
    col_z = g.integers(0, 15, size=N)              # GPTQ zero = nibble + 1 stays <= 15
    p.q = np.broadcast_to(col_q, (K, N)).astype(np.int32)
    p.zq = np.broadcast_to(col_z, (K // 128, N)).astype(np.int32)
    if fmt == AWQ:
        p.qweight = synth.pack_along_n(p.q, awq=True)
        p.qzeros = synth.pack_along_n(p.zq, awq=True)
    else:
        p.qweight = synth.pack_gptq_qweight(p.q)
        p.qzeros = synth.pack_along_n(p.zq, awq=False) if fmt == GPTQ else None
    p.scales = np.full((K // 128, N), 0.5, dtype=np.float16)
    half = np.where(np.arange(K) < K // 2, float(hi), float(lo))
    p.x = (half[None, :] * (2.0 ** -np.arange(M))[:, None]).astype(np.float16)
    c = col_q - p.zero_int()[0]
    assert np.any(np.abs(c) >= 8) and np.any(np.abs(c) < 4)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, 128) == "gemv"
    y = _run_gemm(torch_cuda, p)
    ref = _oracle(orc, p)
    assert np.array_equal(y.astype(np.float64), ref.astype(np.float64)), \
        f"max abs diff {np.max(np.abs(y.astype(np.float64) - ref))}"
    # and again: the hand-off left its slots and masks at zero
    assert np.array_equal(_run_gemm(torch_cuda, p).view(np.uint16), y.view(np.uint16))


@pytest.mark.parametrize("K,N", [(768, 512), (1280, 256), (6144, 1024), (4608, 768),
                                 (4096, 4096), (8192, 1024)])
def test_gemv_awq_m1_tiles(torch_cuda, orc, K, N):
    """AWQ at M = 1 always takes the VALU kernel: the 256-row tile where K % 512 != 0
    (K=768, 1280) or the 512-row tile would leave under 192 workgroups (6144 x 1024, 4608 x
    768, 4096 x 4096), the 512-row tile otherwise (8192 x 1024 would need 32 splits)."""
    p = Problem(AWQ, M=1, K=K, N=N, G=128, seed=1300 + K // 128 + N)
    assert pkg().plan("awq", 1, N, K, 128) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"awq gemv M=1 K={K} N={N}")
    assert np.array_equal(_run_gemm(torch_cuda, p).view(np.uint16), y.view(np.uint16))


@pytest.mark.parametrize("fmt,M,K,N", [(SYM, 1, 16384, 256), (AWQ, 1, 16384, 512),
                                       (AWQ, 8, 2048, 9472), (AWQ, 8, 4096, 14336),
                                       (AWQ, 6, 2048, 14336)])
def test_gemv_split_k_counter_protocol(torch_cuda, orc, fmt, M, K, N):
    """Shapes past the fixed-point hand-off's limits (32 splits; more than 73728 entries
    M * N on the row-paired AWQ kernel) keep the per-tile counter protocol: parity and
    repeatability."""
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=555 + M)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, 128) == "gemv"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"gemv counter protocol fmt={fmt} M={M}")
    assert np.array_equal(_run_gemm(torch_cuda, p).view(np.uint16), y.view(np.uint16))


# ------------------------------------------------------------------ MFMA (small batch / prefill)

@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N", [(5, 1024, 512), (8, 4096, 1024), (16, 512, 256),
                                   (20, 384, 256), (12, 1024, 4096), (32, 512, 4096),
                                   (48, 512, 4096), (33, 1024, 512), (64, 2048, 768), (128, 1024, 512),
                                   (200, 512, 1024)])
def test_mfma_shapes(torch_cuda, orc, fmt, M, K, N):
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=2000 + M + 7 * fmt)
    expect = ("gemv",) if fmt == AWQ and M <= 8 else ("skinny", "prefill")
    assert pkg().plan(FMT_NAME[fmt], M, N, K, p.G) in expect
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"mfma fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt,G", [(AWQ, 32), (AWQ, 64), (GPTQ, 32), (GPTQ, 256), (SYM, 64)])
def test_mfma_group_sizes(torch_cuda, orc, fmt, G):
    p = Problem(fmt, M=24, K=1024, N=512, G=G, seed=2100 + G + fmt)
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"mfma fmt={fmt} G={G}")


@pytest.mark.parametrize("fmt,M,K,N", [
    (AWQ, 8, 4096, 14336),         # config 1, M=8, gate/up
    (AWQ, 8, 14336, 4096),         # config 1, M=8, down
    (GPTQ, 16, 4096, 6144),        # config 2 shape (plain group order)
    (GPTQ, 64, 4096, 6144),
])
def test_mfma_full_size(torch_cuda, orc, fmt, M, K, N):
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED0000 + (1 if fmt == AWQ else 2))
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"full fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt,M,K,N", [
    (GPTQ, 64, 2048, 1024),        # 8 waves, one workgroup per strip
    (SYM, 48, 4096, 2048),         # 8 waves, K split across workgroups
    (GPTQ, 40, 1152, 1024),        # K not a multiple of 256: 4 waves
    (SYM, 64, 384, 512),           # 4 waves
])
def test_small_batch_64_row_tiles_both_wave_counts(torch_cuda, orc, fmt, M, K, N):
    """64-row small-batch tiles run 8 waves (two rounds of LDS reduction) where K is a
    multiple of 256 per split, else 4 waves."""
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED6400 + M + K)
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"64-row tile fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
def test_prefill_full_size_sampled_rows(torch_cuda, orc, K, N):
    """Config 3 (AWQ, M=2048) at full size. The oracle recomputes all 2048 rows of the
    4096 -> 14336 projection (about 15 s on 16 host threads) and 24 sampled rows of the
    14336 -> 4096 one."""
    P = pkg()
    M = 2048
    p = Problem(AWQ, M=M, K=K, N=N, G=128, seed=0x5EED0003)
    assert P.plan("awq", M, N, K, 128) == "prefill"
    y = _run_gemm(torch_cuda, p)
    if (K, N) == (4096, 14336):
        rows = np.arange(M, dtype=np.int32)
    else:
        rows = np.random.default_rng(3).choice(M, 24, replace=False).astype(np.int32)
        rows[:2] = [0, M - 1]
    ref = orc.w4a16_gemm_rows(AWQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prefill K={K} N={N}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("M,K,N", [(1, 4096, 1792), (1, 1792, 4096), (8, 4096, 1792),
                                   (8, 1792, 4096), (2048, 4096, 1792), (2048, 1792, 4096)])
def test_tensor_parallel_shares(torch_cuda, orc, M, K, N):
    """One GPU's share of an 8-way tensor-parallel config-1/3 MLP: the gate/up projection split
    by columns (N = 14336 / 8) and the down projection by rows (K = 14336 / 8). M = 2048 is
    checked on 16 sampled rows."""
    P = pkg()
    p = Problem(AWQ, M=M, K=K, N=N, G=128, seed=0x5EED0100 + M + K)
    assert P.plan("awq", M, N, K, 128) == ("prefill" if M > 64 else "gemv")
    y = _run_gemm(torch_cuda, p)
    if M <= 8:
        assert_parity(y, _oracle(orc, p), what=f"tp share M={M} K={K} N={N}")
        assert np.array_equal(_run_gemm(torch_cuda, p).view(np.uint16), y.view(np.uint16))
        return
    rows = np.random.default_rng(5).choice(M, 16, replace=False).astype(np.int32)
    rows[:2] = [0, M - 1]
    ref = orc.w4a16_gemm_rows(AWQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows)
    assert_parity(y[rows], ref.astype(np.float64), what=f"tp share M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N", [(300, 640, 384), (512, 1024, 128), (2048, 1024, 4096)])
def test_prefill_narrow_tiles(torch_cuda, orc, fmt, M, K, N):
    """256-row x 128-column prefill tiles (two dequantised columns per thread), chosen when
    N is a multiple of 128 but not of 224 or 256, or when they balance the CUs best."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=2300 + M + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, 128) == "prefill"
    y = _run_gemm(torch_cuda, p)
    if M <= 512:
        assert_parity(y, _oracle(orc, p), what=f"prefill 128-wide fmt={fmt} M={M} N={N}")
    else:
        rows = np.random.default_rng(4).choice(M, 16, replace=False).astype(np.int32)
        rows[:2] = [0, M - 1]
        ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows)
        assert_parity(y[rows], ref.astype(np.float64), what=f"prefill 128-wide fmt={fmt} M={M}")


@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N", [(2048, 1024, 6144), (1024, 2048, 6144), (300, 640, 768)])
def test_prefill_192_wide_tiles(torch_cuda, orc, fmt, M, K, N):
    """256 x 192 tiles (widths 224 and 256 do not divide evenly into the CUs: N = 6144 gives
    256 workgroups of 192 columns where 256-wide tiles give 192): unsplit, K split in two
    (M = 1024), and a row tail (M = 300); repeated calls are bit-identical."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=2450 + M + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, 128) == "prefill"
    y = _run_gemm(torch_cuda, p)
    y2 = _run_gemm(torch_cuda, p)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16))
    rows = np.unique(np.r_[0, 255, M - 1, np.random.default_rng(7).choice(M, 16)]).astype(np.int32)
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prefill 192-wide fmt={fmt} M={M} N={N}")


@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N,G", [(2000, 640, 14336, 128), (512, 64, 128, 64),
                                     (512, 192, 128, 64), (1000, 128, 14336, 64)])
def test_prefill_256_row_tiles(torch_cuda, orc, fmt, M, K, N, G):
    """256-row tiles, 224 and 128 columns wide: every format, a row tail, and pipelines of 1,
    2 and 3 stages of 64 k."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=2400 + M + K + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, G) == "prefill"
    y = _run_gemm(torch_cuda, p)
    rows = np.random.default_rng(5).choice(M, 16, replace=False).astype(np.int32)
    rows[:3] = [0, 255, M - 1]
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G, rows)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prefill 256-row tiles fmt={fmt} M={M} K={K}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N", [(512, 2048, 4096), (700, 1024, 2048), (2048, 1024, 4096),
                                   (1024, 14336, 4096), (128, 14336, 4096), (200, 8192, 2048)])
def test_prefill_split_k(torch_cuda, orc, fmt, M, K, N):
    """Few 256-row tiles: K split over workgroups (256 x 128 tiles in 4 and 2 splits, 256 x 128
    unsplit, 256 x 256 in 4 splits, 8 splits where each keeps 16 stages of K), the last split
    of a tile summing the fp32 partials in split order (a row tail included); repeated calls
    are bit-identical."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=2500 + M + fmt)
    assert P.plan(FMT_NAME[fmt], M, N, K, 128) == "prefill"
    y = _run_gemm(torch_cuda, p)
    y2 = _run_gemm(torch_cuda, p)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16))
    rows = np.random.default_rng(6).choice(M, 16, replace=False).astype(np.int32)
    rows[:3] = [0, min(255, M - 1), M - 1]
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows)
    assert_parity(y[rows], ref.astype(np.float64), what=f"prefill split-K fmt={fmt} M={M} N={N}")
    assert np.all(np.isfinite(y))


def test_mfma_split_k_deterministic(torch_cuda, orc):
    P = pkg()
    p = Problem(AWQ, M=8, K=4096, N=1024, G=128, seed=2200)
    args = [to_dev(a) for a in (p.x, p.qweight, p.scales, p.qzeros)]
    ys = [P.gemm(*args, fmt="awq").cpu().numpy() for _ in range(3)]
    assert all(np.array_equal(ys[0].view(np.uint16), y.view(np.uint16)) for y in ys[1:])
    assert_parity(ys[0], _oracle(orc, p))


# ------------------------------------------------------------------ strided / generic

@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
@pytest.mark.parametrize("M,K,N,G", [(16, 384, 264, 128), (64, 960, 392, 64), (37, 384, 200, 128),
                                     (300, 640, 136, 64)])
def test_strided_kernel_via_op(torch_cuda, orc, fmt, M, K, N, G):
    """Shapes the tiled kernels do not take (N not a multiple of their strip, K not of 128)."""
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=1200 + M + fmt)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, p.G) == "strided"
    y = _run_gemm(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"strided fmt={fmt} M={M}")


def test_act_order_gidx(torch_cuda, orc):
    p = Problem(GPTQ, M=16, K=1024, N=384, G=128, seed=1300, act_order=True)
    assert pkg().plan("gptq", p.M, p.N, p.K, p.G, has_g_idx=True) == "skinny"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    assert_parity(y, _oracle(orc, p, g_idx=p.g_idx), what="act-order")


@pytest.mark.parametrize("M", [16, 32, 64])
def test_act_order_config2_full_size(torch_cuda, orc, M):
    """Config 2 at full size: GPTQ act-order, K=4096, N=6144 (fused QKV), G=128."""
    p = Problem(GPTQ, M=M, K=4096, N=6144, G=128, seed=0x5EED0002 + M, act_order=True)
    assert pkg().plan("gptq", M, p.N, p.K, p.G, has_g_idx=True) == "skinny"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    assert_parity(y, _oracle(orc, p, g_idx=p.g_idx), what=f"config 2 M={M}")


@pytest.mark.parametrize("fmt,M,K,N,G,zo", [(SYM, 8, 2048, 512, 128, 1), (GPTQ, 1, 1024, 256, 64, 0),
                                            (GPTQ, 40, 1408, 640, 128, 1), (GPTQ, 5, 512, 64, 32, 1),
                                            (GPTQ, 16, 8192, 256, 32, 1), (SYM, 32, 2048, 512, 32, 1),
                                            (GPTQ, 33, 16384, 3072, 256, 0),
                                            (GPTQ, 16, 4096, 6144, 32, 1), (SYM, 3, 2048, 512, 64, 1)])
def test_act_order_shapes(torch_cuda, orc, fmt, M, K, N, G, zo):
    """Act-order over formats, zero offsets, group sizes, strip widths and split counts; the
    direct-x kernel's (scale, zero) table at its largest (K=4096, G=32, N=6144: 128 groups x
    32 columns) and from 3 rows with G=64.
    K=8192 with G=32 fills the LDS budget with the group table (256 groups), so g_idx is
    read from global memory per step and the table is built after the weight stream is
    issued; the other shapes stage the workgroup's g_idx slice in LDS, K=16384 over two
    splits (8192 rows per workgroup) with the slice loaded after the weight stream."""
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=1310 + M, act_order=True, zero_offset=zo)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, G, has_g_idx=True) == "skinny"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    assert_parity(y, _oracle(orc, p, g_idx=p.g_idx), what=f"act-order fmt={fmt} M={M}")


@pytest.mark.parametrize("M,K,N,G", [(16, 2048, 512, 128), (32, 4096, 1024, 128),
                                     (64, 4096, 768, 256), (48, 2048, 1024, 64),
                                     (16, 4096, 6144, 128)])
def test_act_order_identity_gidx_equals_plain(torch_cuda, orc, M, K, N, G):
    """g_idx[k] = k / G must give the plain result. Act-order runs the direct-x small-batch
    kernel with its per-row (scale, zero) table; plain order runs the same kernel beyond 16
    rows with G a multiple of 128 (per-block scales), and there the output is bit-identical:
    the same per-weight arithmetic and accumulation order. Elsewhere plain order runs the
    split-K kernel: the same bit-exact weights summed in another fp32 order, so the two agree
    to fp16 rounding of equal sums (a few units in the last place) and both meet the oracle."""
    p = Problem(GPTQ, M=M, K=K, N=N, G=G, seed=1320 + M + G)
    assert pkg().plan("gptq", M, N, K, G) == "skinny"
    plain = _run_gemm(torch_cuda, p)
    ident = _run_gemm(torch_cuda, p, g_idx=(np.arange(p.K) // p.G).astype(np.int32))
    if G % 128 == 0 and M > 16:
        assert np.array_equal(plain.view(np.uint16), ident.view(np.uint16))
    else:
        assert_parity(plain, ident.astype(np.float64), tol=2e-3, what="plain vs identity g_idx")
        ref = _oracle(orc, p)
        assert_parity(plain, ref, what="plain")
        assert_parity(ident, ref, what="identity g_idx")


@pytest.mark.parametrize("fmt,M,K,N,G", [(GPTQ, 160, 512, 256, 128), (SYM, 129, 1024, 384, 64),
                                         (GPTQ, 300, 2048, 1024, 256), (GPTQ, 130, 4096, 224, 128),
                                         (GPTQ, 200, 6144, 512, 128), (GPTQ, 72, 8192, 1024, 64),
                                         (GPTQ, 96, 16384, 256, 128), (GPTQ, 150, 1024, 224, 128)])
def test_act_order_large_m_prefill(torch_cuda, orc, fmt, M, K, N, G):
    """Act-order beyond 128 rows (or K beyond 4096) through w4a16_gemm: the group order is
    computed on the device, then the prefill kernel runs on the repacked rows and the gathered
    x (K from 512 to 16384, N from 224 to 1024, groups of 64 to 256 rows)."""
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=1330 + M, act_order=True)
    assert pkg().plan(FMT_NAME[fmt], p.M, p.N, p.K, p.G, has_g_idx=True) == "prefill"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    y2 = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16)), "repeated calls differ"
    assert_parity(y, _oracle(orc, p, g_idx=p.g_idx), what=f"act-order prefill M={M}")


@pytest.mark.parametrize("fmt,M,K,N,G", [(GPTQ, 96, 4096, 6144, 128), (GPTQ, 128, 4096, 6144, 128),
                                         (GPTQ, 65, 1024, 512, 128), (SYM, 100, 2048, 1024, 64),
                                         (GPTQ, 77, 4096, 6144, 32)])
def test_act_order_row_chunks(torch_cuda, orc, fmt, M, K, N, G):
    """Act-order from 65 to 128 rows (K <= 4096): the direct-x small-batch kernel in two row
    chunks, 64 and M - 64, each through its (scale, zero) table; against the oracle, and the
    first 64 rows bit for bit a 64-row call's (each row's sum is its own)."""
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=1390 + M + G, act_order=True)
    assert P.plan(FMT_NAME[fmt], M, N, K, G, has_g_idx=True) == "skinny"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    assert_parity(y, _oracle(orc, p, g_idx=p.g_idx), what=f"act-order row chunks M={M}")
    q = Problem(fmt, M=64, K=K, N=N, G=G, seed=1390 + M + G, act_order=True)
    q.x = p.x[:64].copy()
    q.qweight, q.scales, q.qzeros, q.g_idx = p.qweight, p.scales, p.qzeros, p.g_idx
    y64 = _run_gemm(torch_cuda, q, g_idx=q.g_idx)
    assert np.array_equal(y[:64].view(np.uint16), y64.view(np.uint16))


def test_act_order_config2_prefill_size(torch_cuda, orc):
    """Config 2's act-order weights at M = 2048 (K=4096 -> N=6144): 32 sampled rows."""
    M, K, N = 2048, 4096, 6144
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=0x5EED0002, act_order=True)
    assert pkg().plan("gptq", M, N, K, 128, has_g_idx=True) == "prefill"
    y = _run_gemm(torch_cuda, p, g_idx=p.g_idx)
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(5).choice(M, 30)]).astype(np.int32)
    ref = orc.w4a16_gemm_rows(GPTQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128, rows,
                              g_idx=p.g_idx)
    assert_parity(y[rows], ref.astype(np.float64), what="act-order config 2 M=2048")


def test_act_order_large_m_identity_equals_plain(torch_cuda):
    """g_idx[k] = k / G beyond 64 rows: the group order is the identity, the prefill kernel
    runs on a copy of the same rows and x, so the output is bit for bit the plain call's."""
    p = Problem(GPTQ, M=200, K=1024, N=512, G=128, seed=1335)
    assert pkg().plan("gptq", p.M, p.N, p.K, p.G) == "prefill"
    plain = _run_gemm(torch_cuda, p)
    ident = _run_gemm(torch_cuda, p, g_idx=(np.arange(p.K) // p.G).astype(np.int32))
    assert np.array_equal(plain.view(np.uint16), ident.view(np.uint16))


def test_act_order_large_m_unequal_groups_runs_generic(torch_cuda, orc):
    """A g_idx whose groups do not each hold G rows cannot be put in group order for the
    prefill kernel: the device-side check leaves the generic kernel to run, which reads g_idx
    per row (same results as the oracle)."""
    p = Problem(GPTQ, M=160, K=1024, N=256, G=128, seed=1336)
    assert pkg().plan("gptq", p.M, p.N, p.K, p.G, has_g_idx=True) == "prefill"
    g_idx = np.random.default_rng(1336).integers(0, p.K // p.G, p.K).astype(np.int32)
    g_idx[:5] = 0
    y = _run_gemm(torch_cuda, p, g_idx=g_idx)
    assert_parity(y, _oracle(orc, p, g_idx=g_idx), what="act-order unequal groups")


def test_act_order_large_m_order_kept_between_calls(torch_cuda, orc):
    """Beyond 64 rows the group order computed from g_idx stays on the stream's buffers and is
    reused while g_idx, K and G are unchanged. One stream, calls that change g_idx (another
    order; two rows of different groups swapped; one row moved to another group, so the groups
    are unequal) and then G with the same g_idx (8 groups of 128 rows: valid for G = 128,
    unequal for G = 64), each against the oracle; a repeated g_idx gives its first call's bits."""
    K, N, M = 1024, 256, 160
    p = Problem(GPTQ, M=M, K=K, N=N, G=128, seed=1337, act_order=True)
    assert pkg().plan("gptq", M, N, K, 128, has_g_idx=True) == "prefill"
    p64 = Problem(GPTQ, M=M, K=K, N=N, G=64, seed=1338)
    p64.x = p.x
    rng = np.random.default_rng(1337)
    a = p.g_idx
    b = (np.arange(K) // 128)[rng.permutation(K)].astype(np.int32)
    i = 0
    j = int(np.nonzero(a != a[i])[0][0])
    swapped = a.copy()
    swapped[[i, j]] = a[[j, i]]
    unequal = a.copy()
    unequal[i] = a[j]
    c = (np.arange(K) // 128).astype(np.int32)[::-1].copy()
    first = _run_gemm(torch_cuda, p, g_idx=a)
    assert_parity(first, _oracle(orc, p, g_idx=a), what="g_idx a")
    again = _run_gemm(torch_cuda, p, g_idx=a)
    assert np.array_equal(first.view(np.uint16), again.view(np.uint16)), "repeated g_idx differs"
    for name, g in (("b", b), ("two rows swapped", swapped), ("unequal groups", unequal)):
        y = _run_gemm(torch_cuda, p, g_idx=g)
        assert_parity(y, _oracle(orc, p, g_idx=g), what=f"g_idx {name}")
    y = _run_gemm(torch_cuda, p, g_idx=a)
    assert np.array_equal(first.view(np.uint16), y.view(np.uint16)), "g_idx a after others"
    y = _run_gemm(torch_cuda, p, g_idx=c)
    assert_parity(y, _oracle(orc, p, g_idx=c), what="g_idx c, G=128")
    y = _run_gemm(torch_cuda, p64, g_idx=c)
    assert_parity(y, _oracle(orc, p64, g_idx=c), what="g_idx c, G=64 (unequal groups)")
    y = _run_gemm(torch_cuda, p, g_idx=a)
    assert np.array_equal(first.view(np.uint16), y.view(np.uint16)), "g_idx a after G=64"


@pytest.mark.parametrize("M", [16, 40, 80, 160])
def test_act_order_out_of_range_gidx_is_clamped(torch_cuda, orc, M):
    """The device cannot report a bad g_idx without a host round trip; entries outside
    [0, K/G) are clamped into the scale table (the split-K kernel at 16 rows, the direct-x
    kernel's table offsets at 40 and, in two row chunks, at 80; the oracle, which rejects
    them, is given the clamped index). Beyond 128 rows the group-order check sees them and the
    generic kernel runs."""
    p = Problem(GPTQ, M=M, K=1024, N=256, G=128, seed=1340, act_order=True)
    bad = p.g_idx.copy()
    bad[3], bad[700] = 99, -5
    y = _run_gemm(torch_cuda, p, g_idx=bad)
    ref = _oracle(orc, p, g_idx=np.clip(bad, 0, p.K // p.G - 1).astype(np.int32))
    assert_parity(y, ref, what="clamped g_idx")


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
def test_reference_typed_entry_points_with_strides(torch_cuda, orc, fmt):
    """w4a16_gptq_gemm_typed / awq_gemm_int4_typed with non-contiguous strides and tails."""
    torch = torch_cuda
    P = pkg()
    M, K, N, G = 45, 320, 136, 64
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=1400 + fmt)
    dev = "cuda:0"
    # A stored transposed ([K, M] buffer, read through stride_am=1, stride_ak=M)
    a_t = torch.from_numpy(np.ascontiguousarray(p.x.T)).to(dev)
    # qweight / scales / qzeros with padded leading dimensions
    def padded(a, pad):
        buf = np.zeros((a.shape[0], a.shape[1] + pad), dtype=a.dtype)
        buf[:, : a.shape[1]] = a
        return torch.from_numpy(buf).to(dev), buf.shape[1]
    qw, ldq = padded(p.qweight.view(np.int32), 3)
    sc, lds = padded(p.scales, 5)
    qz, ldz = padded(p.qzeros.view(np.int32), 2)
    c = torch.zeros((M, N + 7), dtype=torch.float16, device=dev)
    fn = P.w4a16_gptq_gemm_typed if fmt == GPTQ else P.awq_gemm_int4_typed
    fn(a_t, qw, sc, qz, c, M, N, K, G, 1, M, ldq, 1, lds, 1, ldz, 1, N + 7, 1)
    torch.cuda.synchronize()
    y = c[:, :N].cpu().numpy()
    ref = _oracle(orc, p)
    assert_parity(y, ref, what="typed strided")
    assert np.all(c[:, N:].cpu().numpy() == 0)   # nothing written outside [M, N]


def test_hip_runtime_module_launch(torch_cuda, orc):
    """DeviceRuntime path: load w4a16_typed.hsaco, launch awq_gemm_int4_typed by name with
    KernelArg values (the reference's 19 parameters + 2 scratch pointers)."""
    torch = torch_cuda
    P = pkg()
    p = Problem(AWQ, M=70, K=256, N=200 // 8 * 8, G=128, seed=1500)
    M, K, N = p.M, p.K, p.N
    rt = P.HipRuntime(0)
    mod = rt.load_module(P.typed_module_bytes())
    meta = {k["name"]: k for k in P.typed_module_meta()["kernels"]}["awq_gemm_int4_typed"]
    a, qw, sc, qz = (to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros))
    c = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
    scratch = torch.empty(1, dtype=torch.uint8, device="cuda:0")
    A = P.KernelArg
    args = [A.ptr(a), A.ptr(qw), A.ptr(sc), A.ptr(qz), A.ptr(c), A.i32(M), A.i32(N), A.i32(K),
            A.i32(p.G), A.i32(K), A.i32(1), A.i32(N // 8), A.i32(1), A.i32(N), A.i32(1),
            A.i32(N // 8), A.i32(1), A.i32(N), A.i32(1), A.ptr(scratch), A.ptr(scratch)]
    grid = (-(-M // meta["block_m"]), -(-N // meta["block_n"]), 1)
    rt.launch(mod, "awq_gemm_int4_typed", grid, (meta["threads_per_block"], 1, 1),
              meta["shared_mem"], None, args)
    torch.cuda.synchronize()
    assert_parity(c.cpu().numpy(), _oracle(orc, p), what="hiprt launch")
    with pytest.raises(P.NotFound):
        rt.launch(mod, "no_such_kernel", grid, (256, 1, 1), 0, None, args)
    with pytest.raises(P.ModuleLoad):
        rt.load_module(b"not a code object at all")
    rt.unload_module(mod)
    rt.close()


def _hiprt_typed_args(P, p, a, qw, sc, qz, c, scratch):
    A = P.KernelArg
    M, K, N = p.M, p.K, p.N
    return [A.ptr(a), A.ptr(qw), A.ptr(sc), A.ptr(qz), A.ptr(c), A.i32(M), A.i32(N), A.i32(K),
            A.i32(p.G), A.i32(K), A.i32(1), A.i32(N // 8 if p.fmt == AWQ else N), A.i32(1), A.i32(N),
            A.i32(1), A.i32(N // 8), A.i32(1), A.i32(N), A.i32(1), A.ptr(scratch), A.ptr(scratch)]


@pytest.mark.parametrize("fmt,M,K,N", [(AWQ, 1, 4096, 14336), (AWQ, 8, 14336, 4096), (GPTQ, 16, 4096, 6144),
                                       (AWQ, 2048, 4096, 14336)])
def test_hip_runtime_launch_planned(torch_cuda, orc, fmt, M, K, N):
    """DeviceRuntime::launch by name at the configs' shapes: a launch of the library's code
    object that follows its contract runs the planned kernels (same results as the C-ABI typed
    entry, bit for bit); a grid off the contract runs the module's own kernel (same function)."""
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=1510 + M)
    rt = P.HipRuntime(0)
    mod = rt.load_module(P.typed_module_bytes())
    name = "awq_gemm_int4_typed" if fmt == AWQ else "w4a16_gptq_gemm_typed"
    a, qw, sc, qz = (to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros))
    c = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
    scratch = torch.empty(1, dtype=torch.uint8, device="cuda:0")
    args = _hiprt_typed_args(P, p, a, qw, sc, qz, c, scratch)
    grid = (-(-M // 64), -(-N // 64), 1)
    rt.launch(mod, name, grid, (256, 1, 1), 0, None, args)
    torch.cuda.synchronize()
    y = c.cpu().numpy()
    fn = P.w4a16_gptq_gemm_typed if fmt == GPTQ else P.awq_gemm_int4_typed
    c2 = torch.empty_like(c)
    fn(a, qw, sc, qz, c2, M, N, K, p.G, K, 1, N // 8 if fmt == AWQ else N, 1, N, 1, N // 8, 1, N, 1)
    torch.cuda.synchronize()
    assert np.array_equal(y.view(np.uint16), c2.cpu().numpy().view(np.uint16)), "hiprt route vs typed entry"
    rows = np.arange(M) if M <= 64 else np.unique(np.r_[0, M - 1, np.random.default_rng(M).choice(M, 30)])
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, p.G, rows.astype(np.int32),
                              zero_offset=p.zero_offset)
    assert_parity(y[rows], ref.astype(np.float64), what=f"hiprt planned {name} M={M}")
    if M <= 16:   # an extra grid row: off the contract, the module's kernel runs
        c.zero_()
        rt.launch(mod, name, (grid[0] + 1, grid[1], 1), (256, 1, 1), 0, None, args)
        torch.cuda.synchronize()
        assert_parity(c.cpu().numpy()[rows], ref.astype(np.float64), what=f"hiprt module kernel {name} M={M}")
    rt.unload_module(mod)
    rt.close()


# ------------------------------------------------------------------ dequant (bit-exact)

@pytest.mark.parametrize("fmt", [GPTQ, SYM, AWQ])
@pytest.mark.parametrize("transposed", [False, True])
def test_dequant_bit_exact(torch_cuda, orc, fmt, transposed):
    P = pkg()
    p = Problem(fmt, M=1, K=512, N=320, G=64, seed=1600 + fmt)
    out = P.dequant(to_dev(p.qweight), to_dev(p.scales),
                    None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt],
                    group_size=p.G, transposed=transposed)
    torch_cuda.cuda.synchronize()
    ref = orc.dequant(fmt, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, transposed=transposed)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_dequant_act_order_bit_exact(torch_cuda, orc):
    P = pkg()
    p = Problem(GPTQ, M=1, K=1024, N=128, G=128, seed=1700, act_order=True)
    out = P.dequant(to_dev(p.qweight), to_dev(p.scales), to_dev(p.qzeros), fmt="gptq",
                    group_size=p.G, g_idx=to_dev(p.g_idx))
    ref = orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, g_idx=p.g_idx)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_reference_dequant_entry_points(torch_cuda, orc):
    """dequant_int4_to_fp16 (zero = nibble, no +1) and dequant_int4_sym_to_fp16, [N, K] output."""
    torch = torch_cuda
    P = pkg()
    K, N, G = 256, 192, 128
    p = Problem(GPTQ, M=1, K=K, N=N, G=G, seed=1800)
    out = torch.empty((N, K), dtype=torch.float16, device="cuda:0")
    P.dequant_int4_to_fp16(to_dev(p.qweight), to_dev(p.scales), to_dev(p.qzeros), out, K, N, G, N // 8)
    ref = orc.dequant(GPTQ, p.qweight, p.scales, p.qzeros, K, N, G, zero_offset=0, transposed=True)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))
    P.dequant_int4_sym_to_fp16(to_dev(p.qweight), to_dev(p.scales), out, K, N, G)
    ref = orc.dequant(SYM, p.qweight, p.scales, None, K, N, G, transposed=True)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))
