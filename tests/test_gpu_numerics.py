"""GPU parity cases that stress the kernels' numerics beyond N(0,1) activations:

* the decode GEMVs apply zero point and scale once per group to a factored fp32 sum,
  s * (sum x (1024 + q) - 1024 sum x - z sum x); with outliers in x and row sums far from
  zero the cancellation error of that form grows with 1024 |sum x|, so these cases check it
  against the oracle's dequant-then-dot (fp64 accumulate) at the benchmark shapes;
* the fixed-point split-K hand-off's fp32 path for partials >= 2^15 on the 256-row tiles the
  GEMVs take for small grids (bit-exact, exact-arithmetic inputs);
* config 1 at M = 4 on the down projection (K = 14336 -> N = 4096) at full size;
* fused-MoE layers of random shapes against the oracle's composition on sampled tokens.
"""
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


def _run(torch, p):
    y = pkg().gemm(to_dev(p.x), to_dev(p.qweight), to_dev(p.scales),
                   None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[p.fmt],
                   group_size=p.G, zero_offset=p.zero_offset)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _oracle(orc, p):
    return orc.w4a16_gemm(p.fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                          zero_offset=p.zero_offset, want_f32=True)[1]


def heavy_tailed_x(g, M, K, n_out=6, mag=300.0, shift=4.0):
    """N(shift, 1) activations (row sums near shift * K, far from zero) with n_out entries
    of +-mag per row, as LLM activations with outlier channels have."""
    x = g.standard_normal((M, K)) + shift
    for m in range(M):
        idx = g.choice(K, n_out, replace=False)
        x[m, idx] = mag * g.choice([-1.0, 1.0], n_out)
    return x.astype(np.float16)


@pytest.mark.parametrize("fmt,M,K,N", [
    (SYM, 1, 4096, 4096),       # config 0 (GPTQ symmetric GEMV)
    (AWQ, 1, 4096, 14336),      # config 1, M = 1 (VALU GEMV, 512-row tiles)
    (AWQ, 1, 14336, 4096),
    (AWQ, 4, 4096, 14336),      # row-paired matrix-core GEMV, fixed-point hand-off
    (AWQ, 8, 4096, 14336),      # row-paired matrix-core GEMV, counter hand-off
    (AWQ, 8, 14336, 4096),      # row-paired matrix-core GEMV, fixed-point hand-off
    (GPTQ, 3, 4096, 6144),      # GPTQ VALU GEMV at M > 1
    (AWQ, 1, 2048, 4096),       # 256-row tiles
])
def test_gemv_heavy_tailed_activations(torch_cuda, orc, fmt, M, K, N):
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED2000 + M + fmt)
    p.x = heavy_tailed_x(np.random.default_rng(0x5EED2100 + M + K), M, K)
    assert pkg().plan(FMT_NAME[fmt], M, N, K, 128) == "gemv"
    y = _run(torch_cuda, p)
    ref = _oracle(orc, p)
    assert np.all(np.isfinite(y))
    assert_parity(y, ref, what=f"heavy-tailed x fmt={fmt} M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt,M,K,N", [(GPTQ, 16, 4096, 6144), (AWQ, 32, 1024, 4096)])
def test_mfma_heavy_tailed_activations(torch_cuda, orc, fmt, M, K, N):
    """The matrix-core kernels dequantise each weight to fp16 exactly (no factored form):
    the same activations stay within the bar there too."""
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED2200 + M)
    p.x = heavy_tailed_x(np.random.default_rng(0x5EED2300 + M), M, K)
    y = _run(torch_cuda, p)
    assert_parity(y, _oracle(orc, p), what=f"heavy-tailed x fmt={fmt} M={M}")


def test_gemv_config1_m4_down_full_size(torch_cuda, orc):
    """Config 1 at M = 4 on the down projection, K = 14336 -> N = 4096 (16 column tiles x 14
    splits of the 1024-row matrix-core tile)."""
    p = Problem(AWQ, M=4, K=14336, N=4096, G=128, seed=0x5EED0001)
    assert pkg().plan("awq", 4, 4096, 14336, 128) == "gemv"
    assert_parity(_run(torch_cuda, p), _oracle(orc, p), what="config 1 M=4 down")


@pytest.mark.parametrize("fmt", [AWQ, GPTQ, SYM])
def test_gemv_256_row_tiles_out_of_range_partials(torch_cuda, orc, fmt):
    """At M = 1, K = 2048, N = 4096 the 512-row tile would leave too few workgroups, so the
    GEMVs run 256-row tiles (8 splits). Exact arithmetic: x = 32 on the first half of K and
    -24 on the second, scales 0.5, q and the zero point constant down each column (c = q - z),
    so a split's partial is 4096 c or -3072 c: >= 2^15 for |c| >= 8 (resp. 11), which takes the
    fixed-point hand-off's fp32 path; the output 4096 c is exact in fp16. Bit-exact against
    the oracle, twice (the hand-off leaves its slots and masks at zero)."""
    K, N = 2048, 4096
    p = Problem(fmt, M=1, K=K, N=N, G=128, seed=5150 + fmt)
    g = np.random.default_rng(5151 + fmt)
    col_q = g.integers(0, 16, size=N)
    col_z = g.integers(0, 15, size=N)
    p.q = np.broadcast_to(col_q, (K, N)).astype(np.int32)
    p.zq = np.broadcast_to(col_z, (K // 128, N)).astype(np.int32)
    if fmt == AWQ:
        p.qweight = synth.pack_along_n(p.q, awq=True)
        p.qzeros = synth.pack_along_n(p.zq, awq=True)
    else:
        p.qweight = synth.pack_gptq_qweight(p.q)
        p.qzeros = synth.pack_along_n(p.zq, awq=False) if fmt == GPTQ else None
    p.scales = np.full((K // 128, N), 0.5, dtype=np.float16)
    p.x = np.where(np.arange(K) < K // 2, 32.0, -24.0)[None, :].astype(np.float16)
    c = col_q - p.zero_int()[0]
    assert np.any(np.abs(c) >= 8) and np.any(np.abs(c) < 8)
    assert pkg().plan(FMT_NAME[fmt], 1, N, K, 128) == "gemv"
    y = _run(torch_cuda, p)
    ref = _oracle(orc, p)
    assert np.array_equal(y.astype(np.float64), ref.astype(np.float64)), \
        f"max abs diff {np.max(np.abs(y.astype(np.float64) - ref))}"
    assert np.array_equal(_run(torch_cuda, p).view(np.uint16), y.view(np.uint16))


def _stacked(fmt, E, K, N, G, seed):
    g = synth.rng(seed)
    shape = (E, K, N // 8) if fmt == AWQ else (E, K // 8, N)
    qw = g.integers(0, 2 ** 32, size=shape, dtype=np.uint32).view(np.int32)
    qz = g.integers(0, 2 ** 32, size=(E, K // G, N // 8), dtype=np.uint32).view(np.int32)
    sc = g.uniform(0.002, 0.02, size=(E, K // G, N)).astype(np.float32).astype(np.float16)
    return qw, sc, qz


def _moe_cases(n=8, seed=4077):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(g.choice([2, 4, 8, 16, 32]))
        topk = int(g.integers(1, min(E, 4) + 1))
        T = int(g.integers(1, 700))
        K = 256 * int(g.integers(1, 5))
        I = 128 * int(g.integers(1, 9))
        out.append((T, E, topk, K, I, int(g.choice([GPTQ, SYM, AWQ]))))
    return out


@pytest.mark.parametrize("case", _moe_cases(), ids=lambda c: "T{}_E{}_k{}_K{}_I{}_f{}".format(*c))
def test_fused_moe_random_layers_vs_oracle(torch_cuda, orc, case):
    """Seeded random layers through w4a16_fused_moe, checked against the oracle's composition
    (route, per-expert dequant-then-matmul, silu*mul, weighted sum) on sampled tokens."""
    torch = torch_cuda
    T, E, topk, K, I, fmt = case
    P = pkg()
    G = 128
    g = np.random.default_rng(T * 13 + E * 5 + I + K)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    w13 = _stacked(fmt, E, K, 2 * I, G, 4093 + T)
    w2 = _stacked(fmt, E, I, K, G, 4094 + T)
    dz = (lambda w: (to_dev(w[0]), to_dev(w[1]), None)) if fmt == SYM else \
         (lambda w: tuple(to_dev(a) for a in w))
    y = P.fused_moe(to_dev(x), to_dev(logits), dz(w13), dz(w2), topk=topk, fmt=FMT_NAME[fmt],
                    group_size=G)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    toks = np.unique(np.concatenate([[0, T - 1], g.choice(T, min(T, 6), replace=False)]))
    ids, w = orc.moe_route(logits, topk)
    z13 = [None if fmt == SYM else w13[2][e] for e in range(E)]
    z2 = [None if fmt == SYM else w2[2][e] for e in range(E)]
    w13d = [orc.dequant(fmt, w13[0][e], w13[1][e], z13[e], K, 2 * I, G) for e in range(E)]
    w2d = [orc.dequant(fmt, w2[0][e], w2[1][e], z2[e], I, K, G) for e in range(E)]
    ref = orc.moe_forward(np.ascontiguousarray(x[toks]), np.ascontiguousarray(ids[toks]),
                          np.ascontiguousarray(w[toks]), w13d, w2d, inter=I)
    assert np.all(np.isfinite(got))
    assert_parity(got[toks], ref.astype(np.float64), what=f"fused moe {case}")
