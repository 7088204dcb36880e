"""GPU tests of the library's robustness contracts: the reference-named typed entry points
reach the planned kernels for dense operands; the split-K workspace outlives the HIP graphs
that captured it; growth under capture is refused before any HIP call; caller-supplied MoE
routing data outside its range is dropped on the device instead of indexing out of bounds;
the silu*mul entry point takes every shape the reference's masked kernel takes."""
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


def _oracle(orc, p, rows=None):
    if rows is None:
        return orc.w4a16_gemm(p.fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G,
                              zero_offset=p.zero_offset, want_f32=True)[1]
    return orc.w4a16_gemm_rows(p.fmt, p.x, p.qweight, p.scales, p.qzeros, p.K, p.N, p.G, rows,
                               zero_offset=p.zero_offset).astype(np.float64)


# ------------------------------------------------------------------ typed entry points

@pytest.mark.parametrize("fmt,M,K,N,expect", [
    (AWQ, 1, 4096, 14336, "gemv"),        # config 1, M=1 (the headline shape)
    (AWQ, 4, 14336, 4096, "gemv"),
    (GPTQ, 16, 4096, 6144, "skinny"),     # config 2 shape, plain group order
    (GPTQ, 1, 4096, 4096, "gemv"),
    (AWQ, 512, 2048, 4096, "prefill"),    # prefill with K split
])
def test_typed_entry_points_dense_take_planned_kernels(torch_cuda, orc, fmt, M, K, N, expect):
    """awq_gemm_int4_typed / w4a16_gptq_gemm_typed with the reference's parameter list and
    dense row-major strides: the plan names the fast kernel, the output equals w4a16_gemm's
    bit for bit (same kernel) and matches the oracle."""
    torch = torch_cuda
    P = pkg()
    p = Problem(fmt, M=M, K=K, N=N, G=128, seed=0x5EED1000 + M + fmt)
    st = [K, 1, N // 8 if fmt == AWQ else N, 1, N, 1, N // 8, 1, N, 1]
    assert P.typed_plan(FMT_NAME[fmt], M, N, K, 128, st) == expect
    a, qw, sc, qz = (to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros))
    c = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
    fn = P.awq_gemm_int4_typed if fmt == AWQ else P.w4a16_gptq_gemm_typed
    fn(a, qw, sc, qz, c, M, N, K, 128, *st)
    y_op = P.gemm(a, qw, sc, qz, fmt=FMT_NAME[fmt], group_size=128, zero_offset=1)
    torch.cuda.synchronize()
    y = c.cpu().numpy()
    assert np.array_equal(y.view(np.uint16), y_op.cpu().numpy().view(np.uint16))
    if M <= 64:
        assert_parity(y, _oracle(orc, p), what=f"typed dense fmt={fmt} M={M}")
    else:
        rows = np.random.default_rng(9).choice(M, 12, replace=False).astype(np.int32)
        assert_parity(y[rows], _oracle(orc, p, rows), what=f"typed dense fmt={fmt} M={M}")


# ------------------------------------------------------------------ workspace and capture

def test_workspace_growth_keeps_captured_graph_valid(torch_cuda, orc):
    """A graph captured with a decode call keeps pointing at the stream's workspace. A later
    eager call that needs a larger workspace (a K-split prefill: 4 x 512 x 4096 fp32
    partials, 32 MiB) must not free that buffer: replays after it, interleaved with eager
    work, still give the oracle's result, bit-identical to the eager call."""
    torch = torch_cuda
    P = pkg()
    s = torch.cuda.Stream()
    p = Problem(AWQ, M=1, K=4096, N=2048, G=128, seed=3100)
    args = [to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros)]
    out = torch.empty((1, p.N), dtype=torch.float16, device="cuda:0")
    with torch.cuda.stream(s):
        P.gemm(*args, fmt="awq", out=out)            # sizes the workspace before capture
    s.synchronize()
    eager = out.cpu().numpy().copy()
    assert_parity(eager, _oracle(orc, p), what="eager decode")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        P.gemm(*args, fmt="awq", out=out)
    q = Problem(AWQ, M=512, K=2048, N=4096, G=128, seed=3101)
    assert P.plan("awq", q.M, q.N, q.K, 128) == "prefill"
    qargs = [to_dev(v) for v in (q.x, q.qweight, q.scales, q.qzeros)]
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            yq = P.gemm(*qargs, fmt="awq")           # grows (first pass) and uses the new workspace
            g.replay()
        s.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), eager.view(np.uint16)), rep
        rows = np.array([0, 100, 511], dtype=np.int32)
        assert_parity(yq.cpu().numpy()[rows], _oracle(orc, q, rows), what="prefill between replays")


def test_workspace_growth_under_capture_is_refused(torch_cuda):
    """A call that would have to allocate a larger workspace while its stream is being captured
    fails on the host (W4A16_ERR_UNSUPPORTED) before any HIP call, leaving the capture intact."""
    torch = torch_cuda
    P = pkg()
    s = torch.cuda.Stream()                          # fresh stream: no workspace yet
    p = Problem(AWQ, M=1, K=4096, N=2048, G=128, seed=3102)
    args = [to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(P.Unsupported, match="before capturing"):
        with torch.cuda.graph(g, stream=s):
            P.gemm(*args, fmt="awq")
    # the same call outside capture works and sizes the workspace
    with torch.cuda.stream(s):
        y = P.gemm(*args, fmt="awq")
    s.synchronize()
    assert np.all(np.isfinite(y.cpu().numpy()))


def test_init_then_capture_replays(torch_cuda, orc):
    """w4a16_init before capture; a decode GEMV captured once and replayed several times with
    eager work in between matches the oracle on every replay."""
    torch = torch_cuda
    P = pkg()
    P.init(0)
    s = torch.cuda.Stream()
    p = Problem(GPTQ, M=2, K=2048, N=1024, G=128, seed=3103)
    args = [to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros)]
    out = torch.empty((2, p.N), dtype=torch.float16, device="cuda:0")
    with torch.cuda.stream(s):
        P.gemm(*args, fmt="gptq", out=out)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        P.gemm(*args, fmt="gptq", out=out)
    ref = _oracle(orc, p)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_parity(out.cpu().numpy(), ref, what="captured decode replay")


def test_captured_graph_of_each_kernel_family_replays_exactly(torch_cuda):
    """One graph holding a call of each kernel family with its split-K state: the row-paired
    AWQ GEMV (fixed-point hand-off), the act-order small-batch kernel (group table and g_idx
    slice in LDS; 16 rows with 4 waves, 64 rows with 8 waves and K split in two), a K-split
    prefill (fp32 partials, counter hand-off) and the prepared
    act-order path (LDS column gather, then the small-batch kernel). Replayed three times with
    other eager calls on the same stream in between, every replay equals the eager outputs bit
    for bit (the hand-offs leave their counters and slots clean; the launch-time LDS
    allowances are valid under capture)."""
    torch = torch_cuda
    P = pkg()
    s = torch.cuda.Stream()
    cases = [
        (Problem(AWQ, M=4, K=4096, N=2048, G=128, seed=3110), "awq", False, False),
        (Problem(GPTQ, M=16, K=2048, N=1024, G=128, seed=3111, act_order=True), "gptq", True, False),
        (Problem(AWQ, M=512, K=2048, N=4096, G=128, seed=3112), "awq", False, False),
        (Problem(GPTQ, M=64, K=2048, N=1024, G=128, seed=3113, act_order=True), "gptq", True, True),
        # 64-row act-order tile of 8 waves with K split in two (counter hand-off)
        (Problem(GPTQ, M=64, K=4096, N=1024, G=128, seed=3115, act_order=True), "gptq", True, False),
    ]
    assert P.plan("awq", 512, 4096, 2048, 128) == "prefill"
    calls = []
    for p, fmt, act, prepared in cases:
        x, qw, sc, qz = (to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros))
        gi = to_dev(p.g_idx) if act else None
        out = torch.empty((p.M, p.N), dtype=torch.float16, device="cuda:0")
        if prepared:
            qp, perm = P.prepare_act_order(qw, gi, group_size=p.G)
            calls.append(lambda x=x, qp=qp, sc=sc, qz=qz, perm=perm, out=out, G=p.G:
                         P.gemm_act_order(x, qp, sc, qz, perm, group_size=G, out=out))
        else:
            calls.append(lambda x=x, qw=qw, sc=sc, qz=qz, gi=gi, out=out, fmt=fmt, G=p.G:
                         P.gemm(x, qw, sc, qz, fmt=fmt, group_size=G, g_idx=gi, out=out))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):                        # eager: sizes the stream's buffers
        outs = [c() for c in calls]
    s.synchronize()
    eager = [o.cpu().numpy().copy() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for c in calls:
            c()
    other = Problem(AWQ, M=8, K=2048, N=4096, G=128, seed=3114)
    oargs = [to_dev(v) for v in (other.x, other.qweight, other.scales, other.qzeros)]
    for rep in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            P.gemm(*oargs, fmt="awq")                 # eager split-K work between replays
            g.replay()
            P.gemm(*oargs, fmt="awq")
        s.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert np.array_equal(o.cpu().numpy().view(np.uint16), e.view(np.uint16)), (rep, i)


def test_concurrent_streams_and_threads_keep_split_k_state_apart(torch_cuda):
    """Split-K calls on two streams at once, issued from two host threads: each stream has its
    own workspace (counters, fixed-point slots, partials), so the interleaved calls give the
    single-stream outputs bit for bit (a decode GEMV with the fixed-point hand-off on one
    stream, a small-batch GEMM with the counter hand-off on the other)."""
    import threading
    torch = torch_cuda
    P = pkg()
    pa = Problem(AWQ, M=1, K=4096, N=4096, G=128, seed=3120)
    pb = Problem(GPTQ, M=16, K=2048, N=2048, G=128, seed=3121)
    aa = [to_dev(v) for v in (pa.x, pa.qweight, pa.scales, pa.qzeros)]
    ab = [to_dev(v) for v in (pb.x, pb.qweight, pb.scales, pb.qzeros)]
    ref_a = P.gemm(*aa, fmt="awq").cpu().numpy()
    ref_b = P.gemm(*ab, fmt="gptq").cpu().numpy()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    outs_a = [torch.empty((pa.M, pa.N), dtype=torch.float16, device="cuda:0") for _ in range(20)]
    outs_b = [torch.empty((pb.M, pb.N), dtype=torch.float16, device="cuda:0") for _ in range(20)]
    torch.cuda.synchronize()
    errors = []

    def run(stream, args, fmt, outs):
        try:
            with torch.cuda.stream(stream):
                for o in outs:
                    P.gemm(*args, fmt=fmt, out=o)
            stream.synchronize()
        except Exception as e:   # reported by the main thread
            errors.append(e)

    ta = threading.Thread(target=run, args=(sa, aa, "awq", outs_a))
    tb = threading.Thread(target=run, args=(sb, ab, "gptq", outs_b))
    ta.start(); tb.start(); ta.join(); tb.join()
    assert not errors, errors
    for o in outs_a:
        assert np.array_equal(o.cpu().numpy().view(np.uint16), ref_a.view(np.uint16))
    for o in outs_b:
        assert np.array_equal(o.cpu().numpy().view(np.uint16), ref_b.view(np.uint16))


def test_python_wrappers_reject_bad_layouts_before_launch(torch_cuda):
    """The C ABI takes contiguous row-major buffers: the Python wrappers of every GEMM entry
    point refuse a transposed view, a wrong dtype or a missing output before any launch."""
    torch = torch_cuda
    P = pkg()
    p = Problem(GPTQ, M=4, K=256, N=256, G=128, seed=0x5EED5000)
    x, qw, sc, qz = (to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros))
    x_t = torch.empty((p.K, p.M), dtype=torch.float16, device="cuda:0").t()
    perm = torch.arange(p.K, dtype=torch.int32, device="cuda:0")
    out = torch.empty((p.M, p.N), dtype=torch.float16, device="cuda:0")
    with pytest.raises(P.InvalidArgument, match="x must be contiguous"):
        P.gemm(x_t, qw, sc, qz, fmt="gptq")
    with pytest.raises(P.InvalidArgument, match="x must be contiguous"):
        P.gemm_act_order(x_t, qw, sc, qz, perm)
    with pytest.raises(P.InvalidArgument, match="x must be contiguous"):
        P.gemm_noalloc(x_t, qw, sc, qz, out, fmt="gptq")
    with pytest.raises(P.InvalidArgument, match="perm has dtype"):
        P.gemm_act_order(x, qw, sc, qz, perm.long())
    with pytest.raises(P.InvalidArgument, match="scales has dtype"):
        P.gemm_noalloc(x, qw, sc.float(), qz, out, fmt="gptq")
    with pytest.raises(P.InvalidArgument, match="out must be given"):
        P.gemm_noalloc(x, qw, sc, qz, None, fmt="gptq")
    with pytest.raises(P.InvalidArgument, match="out must be a contiguous"):
        P.gemm_act_order(x, qw, sc, qz, perm, out=out.t().contiguous())
    with pytest.raises(P.InvalidArgument, match="qweight must be contiguous"):
        P.dequant(qw.t().contiguous().t(), sc, qz, fmt="gptq")


# ------------------------------------------------------------------ MoE routing data

def test_align_drops_out_of_range_expert_ids(torch_cuda, orc):
    """topk_ids outside [0, E) are dropped by the align kernel (no out-of-bounds access); the
    valid pairs are placed exactly as the oracle places them when the bad pairs are absent."""
    P = pkg()
    T, E, topk, bm = 200, 8, 2, 64
    g = np.random.default_rng(3200)
    ids, _ = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    bad = ids.copy().ravel()
    bad[[3, 50, 51, 399]] = [8, -1, 1 << 20, -(1 << 30)]
    sorted_ids, expert_ids, npp = P.moe_align(to_dev(bad.reshape(T, topk)), E, bm)
    n = int(npp.cpu().numpy()[0])
    got = sorted_ids.cpu().numpy()[:n]
    keep = (bad >= 0) & (bad < E)
    # the oracle on the valid pairs only, with their original pair indices
    s_ref = []
    for e in range(E):
        pairs = np.nonzero(keep & (bad == e))[0]
        pad = (-len(pairs)) % bm
        s_ref.extend(list(pairs) + [T * topk] * pad)
    assert n == len(s_ref)
    assert np.array_equal(got, np.array(s_ref, dtype=np.int32))
    assert not np.isin([3, 50, 51, 399], got).any()


def test_grouped_gemm_skips_out_of_range_expert_and_pair_ids(torch_cuda, orc):
    """A block whose expert id is outside [0, num_experts) is skipped and a sorted id outside
    [0, num_pairs) is padding: their output rows keep the sentinel value, the other rows are
    correct."""
    torch = torch_cuda
    P = pkg()
    T, E, topk, K, N, G, bm = 40, 4, 2, 256, 512, 128, 64
    g = np.random.default_rng(3201)
    x = synth.rand_x(g, T, K)
    ids, _ = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    shape = (E, K // 8, N)
    qw = g.integers(0, 2 ** 32, size=shape, dtype=np.uint32).view(np.int32)
    qz = g.integers(0, 2 ** 32, size=(E, K // G, N // 8), dtype=np.uint32).view(np.int32)
    sc = g.uniform(0.002, 0.02, size=(E, K // G, N)).astype(np.float32).astype(np.float16)
    sorted_ids, expert_ids, npp = P.moe_align(to_dev(ids), E, bm)
    e_host = expert_ids.cpu().numpy().copy()
    s_host = sorted_ids.cpu().numpy().copy()
    n = int(npp.cpu().numpy()[0])
    bad_block = 0
    e_host[bad_block] = E + 3                          # whole block skipped
    victim_pos = n - 1 if s_host[n - 1] < T * topk else int(np.nonzero(s_host[:n] < T * topk)[0][-1])
    victim = int(s_host[victim_pos])
    s_host[victim_pos] = -7                            # treated as padding
    out = torch.full((T * topk, N), 12345.0, dtype=torch.float16, device="cuda:0")
    P.moe_gemm(to_dev(x), topk, to_dev(qw), to_dev(sc), to_dev(qz), to_dev(s_host), to_dev(e_host),
               npp, T * topk, N, K, fmt="gptq", group_size=G, block_m=bm, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    skipped = set(int(v) for v in s_host[bad_block * bm:(bad_block + 1) * bm] if 0 <= v < T * topk)
    skipped.add(victim)
    for pr in range(T * topk):
        if pr in skipped:
            assert np.all(got[pr] == 12345.0), pr
    for e in range(E):
        pairs = [pr for pr in np.nonzero(ids.ravel() == e)[0] if pr not in skipped]
        if not pairs:
            continue
        pairs = np.array(pairs)
        ref = orc.w4a16_gemm(GPTQ, np.ascontiguousarray(x[pairs // topk]), qw[e], sc[e], qz[e], K,
                             N, G, want_f32=True)[1]
        assert_parity(got[pairs], ref, what=f"expert {e}")


# ------------------------------------------------------------------ silu * mul

@pytest.mark.parametrize("rows,inter,total_cut,offset", [
    (33, 1024, 0, 0),      # four outputs per thread
    (7, 100, 0, 0),        # inter a multiple of 4, not of 8
    (5, 1023, 0, 0),       # odd inter
    (5, 1024, 0, 1),       # unaligned pointers (one element in)
    (6, 96, 37, 0),        # total not a multiple of inter: the last row cut short
    (3, 1, 0, 0),
])
def test_silu_mul_f32_entry_point(torch_cuda, orc, rows, inter, total_cut, offset):
    """fused_silu_mul_interleaved_f32 (elementwise.rs:214-250) against the oracle: both compute
    exp(-g) + 1, a division and a product in f32; the device and host expf may differ by an
    ulp, which moves the result by a few f32 ulps at most."""
    torch = torch_cuda
    P = pkg()
    g = np.random.default_rng(3400 + inter + offset)
    gu = (g.standard_normal((rows, 2 * inter)) * 4).astype(np.float32)
    special = np.array([0.0, 100.0, -100.0, 30.0], dtype=np.float32)   # zero, saturation,
    gu[0, :min(4, inter)] = special[:min(4, inter)]                    # overflow of exp(-g)
    total = rows * inter - total_cut
    buf = torch.zeros(rows * 2 * inter + offset, dtype=torch.float32, device="cuda:0")
    buf[offset:] = torch.from_numpy(gu.ravel()).to("cuda:0")
    obuf = torch.full((rows * inter + offset,), -7.0, dtype=torch.float32, device="cuda:0")
    P.fused_silu_mul_interleaved_f32(buf[offset:], obuf[offset:], inter, total)
    torch.cuda.synchronize()
    got = obuf.cpu().numpy()[offset:].astype(np.float64)
    ref = orc.silu_mul_f32_rows(gu, inter, total).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got[:total] - ref) <= 4 * ulp + 1e-37)
    assert np.mean(got[:total] == ref) > 0.9
    assert np.all(got[total:] == -7.0)               # nothing written past `total`


@pytest.mark.parametrize("rows,inter,total_cut,offset", [
    (7, 100, 0, 0),        # inter not a multiple of 8
    (5, 1024, 0, 1),       # unaligned pointers (one element in)
    (6, 96, 37, 0),        # total not a multiple of inter: the last row cut short
    (3, 1, 0, 0),
])
def test_silu_mul_any_shape(torch_cuda, orc, rows, inter, total_cut, offset):
    torch = torch_cuda
    P = pkg()
    g = np.random.default_rng(3300 + inter)
    gu = (g.standard_normal((rows, 2 * inter)) * 3).astype(np.float16)
    total = rows * inter - total_cut
    buf = torch.zeros(rows * 2 * inter + offset, dtype=torch.float16, device="cuda:0")
    buf[offset:] = torch.from_numpy(gu.ravel()).to("cuda:0")
    obuf = torch.full((rows * inter + offset,), -7.0, dtype=torch.float16, device="cuda:0")
    P.fused_silu_mul_interleaved_f16(buf[offset:], obuf[offset:], inter, total)
    torch.cuda.synchronize()
    got = obuf.cpu().numpy()[offset:].astype(np.float64)
    ref = orc.silu_mul_f16(gu[:, :inter], gu[:, inter:]).ravel().astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got[:total] - ref[:total]) <= ulp[:total] + 1e-7)
    assert np.all(got[total:] == -7.0)               # nothing written past `total`


def test_captured_graph_of_act_order_prefill_route(torch_cuda, orc):
    """The act-order route beyond 64 rows under graph capture: two layers with different g_idx
    on one stream (the group order kept on the stream's buffers changes on every call) and one
    whose groups are unequal (the generic kernel runs). Three replays, with eager calls on the
    stream in between, each give the eager outputs bit for bit; then one layer's g_idx is
    rewritten in place and the next replay follows the new order (its output equals an eager
    call with it, and the oracle)."""
    torch = torch_cuda
    P = pkg()
    s = torch.cuda.Stream()
    K, N, M, G = 1024, 256, 160, 128
    pa = Problem(GPTQ, M=M, K=K, N=N, G=G, seed=3130, act_order=True)
    pb = Problem(GPTQ, M=M, K=K, N=N, G=G, seed=3131, act_order=True)
    pc = Problem(GPTQ, M=M, K=K, N=N, G=G, seed=3132)
    assert P.plan("gptq", M, N, K, G, has_g_idx=True) == "prefill"
    gc = np.random.default_rng(3132).integers(0, K // G, K).astype(np.int32)
    layers = []
    for p, gi in ((pa, pa.g_idx), (pb, pb.g_idx), (pc, gc)):
        args = [to_dev(v) for v in (p.x, p.qweight, p.scales, p.qzeros)]
        layers.append((args, to_dev(gi), torch.empty((M, N), dtype=torch.float16, device="cuda:0")))

    def run(i):
        (x, qw, sc, qz), gi, out = layers[i]
        P.gemm(x, qw, sc, qz, fmt="gptq", group_size=G, g_idx=gi, out=out)

    torch.cuda.synchronize()
    with torch.cuda.stream(s):                        # eager: sizes the stream's buffers
        for i in range(3):
            run(i)
    s.synchronize()
    eager = [o.cpu().numpy().copy() for _, _, o in layers]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(3):
            run(i)
    for rep in range(3):
        for _, _, o in layers:
            o.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            run(1)                                    # eager act-order work between replays
            g.replay()
        s.synchronize()
        for i, (_, _, o) in enumerate(layers):
            assert np.array_equal(o.cpu().numpy().view(np.uint16), eager[i].view(np.uint16)), (rep, i)
    new = (np.arange(K) // G)[np.random.default_rng(3133).permutation(K)].astype(np.int32)
    with torch.cuda.stream(s):
        layers[0][1].copy_(torch.from_numpy(new).to("cuda:0"))
        g.replay()
    s.synchronize()
    replayed = layers[0][2].cpu().numpy().copy()
    with torch.cuda.stream(s):
        run(0)
    s.synchronize()
    assert np.array_equal(replayed.view(np.uint16), layers[0][2].cpu().numpy().view(np.uint16))
    ref = orc.w4a16_gemm(GPTQ, pa.x, pa.qweight, pa.scales, pa.qzeros, K, N, G, g_idx=new,
                         want_f32=True)[1]
    assert_parity(replayed, ref, what="replay after g_idx rewritten")
