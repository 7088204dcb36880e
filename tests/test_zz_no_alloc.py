"""w4a16_gemm_noalloc, the allocation-free variant of w4a16_gemm (its split-K scratch is a
fixed per-device array): through the C ABI, against w4a16_gemm on the same inputs, on two
calls in a row with the second smaller, plus its size limit. Runs alone in a fresh process
(the first call sets the device's array up) and after the other tests."""
import ctypes

import numpy as np
import pytest

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


def _call(P, torch, fn, p, g_idx=None):
    L = P.lib()
    x, qw, sc = to_dev(p.x), to_dev(p.qweight), to_dev(p.scales)
    qz = None if p.qzeros is None else to_dev(p.qzeros)
    gi = None if g_idx is None else to_dev(g_idx)
    out = torch.full((p.M, p.N), 777.0, dtype=torch.float16, device="cuda:0")
    ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(L, fn)(st, p.fmt, ptr(x), ptr(qw), ptr(sc), ptr(qz), ptr(gi), ptr(out), p.M, p.N,
                        p.K, p.G, p.zero_offset)
    torch.cuda.synchronize()
    return rc, out.cpu().numpy()


# (first call, second call with a smaller input) per kernel regime
PAIRS = [
    ((AWQ, 1, 4096, 14336, False), (AWQ, 1, 1024, 512, False)),     # VALU GEMV, fixed-point
    ((GPTQ, 4, 4096, 6144, False), (SYM, 1, 2048, 1024, False)),     # GPTQ GEMV
    ((AWQ, 8, 4096, 14336, False), (AWQ, 6, 2048, 1024, False)),     # matrix-core GEMV, counter
    ((GPTQ, 64, 4096, 6144, True), (GPTQ, 16, 1024, 768, True)),     # small batch, act-order
    ((GPTQ, 96, 4096, 6144, True), (GPTQ, 70, 1024, 768, True)),     # act-order in row chunks
    ((AWQ, 512, 2048, 4096, False), (GPTQ, 300, 640, 384, False)),   # prefill (K split > scratch)
]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda c: "{}_M{}_K{}_N{}_g{}".format(*c[0]))
def test_noalloc_matches_w4a16_gemm(torch_cuda, orc, pair):
    torch = torch_cuda
    P = pkg()
    for i, (fmt, M, K, N, act) in enumerate(pair):
        p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED3000 + 10 * i + M, act_order=act)
        rc_na, y_na = _call(P, torch, "w4a16_gemm_noalloc", p, p.g_idx)
        assert rc_na == P.OK, P.lib().w4a16_last_error()
        rc, y = _call(P, torch, "w4a16_gemm", p, p.g_idx)
        assert rc == P.OK
        same_plan = not (M > 64 and P.plan(FMT_NAME[fmt], M, N, K, 128, has_g_idx=act) == "prefill")
        if same_plan:
            # same kernels, same deterministic split-K order: the same bits
            assert np.array_equal(y_na.view(np.uint16), y.view(np.uint16)), (fmt, M, K, N)
        else:
            # the prefill's K split needs more than the fixed scratch: it runs with fewer
            # splits, or none
            assert_parity(y_na, y.astype(np.float64), what=f"noalloc prefill M={M}")
        rows = np.arange(M) if M <= 64 else np.array([0, M // 2, M - 1])
        ref = orc.w4a16_gemm_rows(fmt, p.x, p.qweight, p.scales, p.qzeros, K, N, 128,
                                  rows.astype(np.int32), g_idx=p.g_idx,
                                  zero_offset=p.zero_offset).astype(np.float64)
        assert_parity(y_na[rows], ref, what=f"noalloc fmt={fmt} M={M} K={K} N={N}")
        # and repeated: the kernels left the shared array's counters and slots at zero
        rc_na, y_na2 = _call(P, torch, "w4a16_gemm_noalloc", p, p.g_idx)
        assert rc_na == P.OK
        assert np.array_equal(y_na2.view(np.uint16), y_na.view(np.uint16))


@pytest.mark.parametrize("K,N", [(16384, 16384), (8192, 28672), (28672, 8192)])
def test_noalloc_beyond_its_scratch_runs_a_smaller_split(torch_cuda, orc, K, N):
    """AWQ M=8 whose split-K partials exceed the 6.9 MiB the fixed array holds (K=16384 ->
    N=16384: 8 MiB; a 70B-class MLP, 8192 -> 28672 and 28672 -> 8192: 7 MiB): the call is
    re-planned onto the prefill kernel with the largest K split whose partials fit the array
    (at most 8 x 8 x 16384 fp32 = 4 MiB here; none needs no scratch at all), and matches
    the oracle and w4a16_gemm within the tolerance; then a small call through the split-K
    GEMV still gives w4a16_gemm's bits (the array was left clean)."""
    torch = torch_cuda
    P = pkg()
    assert P.lib().w4a16_gemm_noalloc_scratch_bytes() == 8 << 20
    p = Problem(AWQ, M=8, K=K, N=N, G=128, seed=0x5EED3100 + K)
    rc, y = _call(P, torch, "w4a16_gemm_noalloc", p)
    assert rc == P.OK, P.lib().w4a16_last_error()
    rc, y_ref = _call(P, torch, "w4a16_gemm", p)
    assert rc == P.OK
    assert_parity(y, y_ref.astype(np.float64), what=f"noalloc vs w4a16_gemm K={K} N={N}")
    ref = orc.w4a16_gemm_rows(AWQ, p.x, p.qweight, p.scales, p.qzeros, K, N, 128,
                              np.arange(8, dtype=np.int32), zero_offset=0).astype(np.float64)
    assert_parity(y, ref, what=f"noalloc M=8 K={K} N={N}")
    q = Problem(AWQ, M=1, K=4096, N=14336, G=128, seed=0x5EED3101)
    rc_na, y_na = _call(P, torch, "w4a16_gemm_noalloc", q)
    rc, y = _call(P, torch, "w4a16_gemm", q)
    assert rc_na == P.OK and rc == P.OK
    assert np.array_equal(y_na.view(np.uint16), y.view(np.uint16))
