"""GPU parity over seeded random shapes: every GEMM regime the dispatcher can pick (VALU and
matrix-core GEMV, small batch with and without act-order, prefill with and without split K,
generic strided kernel), with K, N, group size and format drawn together, checked against
the CPU oracle on sampled rows. The draws are fixed by the seed, so a failure names its
case and reproduces on the CPU oracle side."""
import os

import numpy as np
import pytest

from helpers import assert_parity, pkg, to_dev
from synth import Problem

pytestmark = pytest.mark.gpu
FMT_NAME = {0: "gptq", 1: "gptq_sym", 2: "awq"}


def _draw_cases(n=80, seed=20261202):
    g = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        fmt = int(g.integers(0, 3))
        band = int(g.integers(0, 3))
        M = int(g.integers(1, 9)) if band == 0 else int(g.integers(9, 65)) if band == 1 \
            else int(g.integers(65, 1100))
        G = int(g.choice([32, 64, 128]))
        # mostly the tile-friendly sizes the fast kernels take, sometimes any multiple
        K = 256 * int(g.integers(1, 17)) if g.random() < 0.7 else \
            G * int(g.integers(max(1, 128 // G), 4096 // G + 1))
        N = 8 * int(g.integers(8, 513)) if g.random() < 0.25 else 256 * int(g.integers(1, 17))
        act_order = fmt != 2 and M <= 64 and g.random() < 0.3
        if M * N * K > 2_000_000_000:
            continue
        cases.append((fmt, M, K, N, G, act_order))
    return cases


# W4A16_RANDOM_CASES / W4A16_RANDOM_SEED widen the sweep for a longer run (defaults: the
# committed 80 cases)
CASES = _draw_cases(int(os.environ.get("W4A16_RANDOM_CASES", "80")),
                    int(os.environ.get("W4A16_RANDOM_SEED", "20261202")))


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("case", CASES, ids=[f"{FMT_NAME[c[0]]}-M{c[1]}-K{c[2]}-N{c[3]}-G{c[4]}"
                                             f"{'-ao' if c[5] else ''}" for c in CASES])
def test_random_shape_matches_oracle(torch_cuda, orc, case):
    fmt, M, K, N, G, ao = case
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=G, seed=(fmt * 1000003 + M * 7919 + K * 31 + N) & 0xFFFF,
                act_order=ao)
    kernel = P.plan(FMT_NAME[fmt], M, N, K, G, has_g_idx=ao)
    assert kernel in ("gemv", "skinny", "prefill", "strided")
    y = P.gemm(to_dev(p.x), to_dev(p.qweight), to_dev(p.scales),
               None if p.qzeros is None else to_dev(p.qzeros), fmt=FMT_NAME[fmt], group_size=G,
               g_idx=None if p.g_idx is None else to_dev(p.g_idx), zero_offset=p.zero_offset)
    torch_cuda.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M + K + N).integers(0, M, 6)]))
    rows = rows.astype(np.int32)
    ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, G, rows,
                              g_idx=p.g_idx, zero_offset=p.zero_offset)
    assert_parity(y[rows], ref.astype(np.float64), what=f"{case} ({kernel})")
    assert np.all(np.isfinite(y))
