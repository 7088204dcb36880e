"""Exact-arithmetic known answers (tests/golden/exact_gemm.npz, made by make_exact_gemm.py).

Every dequantised weight, product and partial sum of these cases is exact in fp32, so a
correct GEMM returns the exact sum rounded once to fp16 whatever its accumulation order:
the oracle and every kernel regime must match the fixture bit for bit. The fixture is
computed with integer arithmetic only, independently of the oracle and of the kernels.
"""
import os

import numpy as np
import pytest

from helpers import pkg

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "exact_gemm.npz")
FMT_NAME = {0: "gptq", 1: "gptq_sym", 2: "awq"}
EXPECT_KERNEL = {
    "awq_m1_k512_n256": "gemv", "gptq_m1_k512_n256": "gemv", "sym_m3_k512_n128": "gemv",
    "awq_m8_k512_n256": "gemv", "gptq_m16_k512_n256": "skinny", "awq_m24_k512_n256": "skinny",
    "gptq_ao_m16_k512_n256": "skinny", "gptq_m128_k256_n256": "prefill",
    "awq_m96_k256_n384": "prefill", "awq_m5_k384_n200": "strided",
    "awq_m6_k1024_n256": "gemv",
}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _cases():
    d = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in d.files})
    return d, names


def _case(d, name):
    fmt, M, K, N, G, ao = (int(v) for v in d[name + "/meta"])
    g_idx = d[name + "/g_idx"] if ao else None
    return (fmt, M, K, N, G, d[name + "/x"], d[name + "/qweight"], d[name + "/scales"],
            d[name + "/qzeros"], g_idx, d[name + "/out"])


def test_golden_file_covers_every_regime():
    d, names = _cases()
    assert set(names) == set(EXPECT_KERNEL)
    P = pkg()
    for name in names:
        fmt, M, K, N, G, *_ = _case(d, name)
        ao = int(d[name + "/meta"][5])
        assert P.plan(FMT_NAME[fmt], M, N, K, G, has_g_idx=bool(ao)) == EXPECT_KERNEL[name], name


@pytest.mark.parametrize("name", sorted(EXPECT_KERNEL))
def test_oracle_matches_exact_answers(orc, name):
    d, _ = _cases()
    fmt, M, K, N, G, x, qw, sc, qz, g_idx, out = _case(d, name)
    y = orc.w4a16_gemm(fmt, x, qw, sc, qz, K, N, G, g_idx=g_idx)
    assert np.array_equal(y.view(np.uint16), out), name


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(EXPECT_KERNEL))
def test_gpu_matches_exact_answers(torch_cuda, name):
    torch = torch_cuda
    d, _ = _cases()
    fmt, M, K, N, G, x, qw, sc, qz, g_idx, out = _case(d, name)
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    P = pkg()
    y = P.gemm(t(x.view(np.float16)), t(qw), t(sc.view(np.float16)),
               t(qz) if fmt != 1 else None, fmt=FMT_NAME[fmt], group_size=G,
               g_idx=t(g_idx) if g_idx is not None else None)
    got = y.cpu().numpy().view(np.uint16)
    diff = np.argwhere(got != out)
    assert diff.size == 0, (f"{name} ({EXPECT_KERNEL[name]}): {len(diff)} of {out.size} outputs "
                            f"differ, first at {diff[0].tolist()}: got {got[tuple(diff[0])]:#06x} "
                            f"want {out[tuple(diff[0])]:#06x}")
