"""GPU parity of the fused-MoE path (route, align, grouped GEMM, silu*mul, combine, whole
layer) against the CPU oracle. The reference has no MoE kernel; the oracle defines the
layer by composition of the pinned dense pieces (tests/test_oracle.py::test_moe_*)."""
import numpy as np
import pytest

import synth
from helpers import assert_parity, pkg, to_dev

pytestmark = pytest.mark.gpu
GPTQ, SYM, AWQ = 0, 1, 2
FMT_NAME = {GPTQ: "gptq", SYM: "gptq_sym", AWQ: "awq"}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def stacked_weights(fmt, E, K, N, G, seed):
    """Per-expert packed weights stacked along a leading expert dimension. Uniform random
    32-bit words are uniform nibbles in every slot, so the words are drawn directly."""
    g = synth.rng(seed)
    shape = (E, K, N // 8) if fmt == AWQ else (E, K // 8, N)
    qw = g.integers(0, 2 ** 32, size=shape, dtype=np.uint32).view(np.int32)
    qz = g.integers(0, 2 ** 32, size=(E, K // G, N // 8), dtype=np.uint32).view(np.int32)
    sc = g.uniform(0.002, 0.02, size=(E, K // G, N)).astype(np.float32).astype(np.float16)
    return qw, sc, qz


def test_route_matches_oracle(torch_cuda, orc):
    P = pkg()
    g = np.random.default_rng(70)
    for T, E, topk in ((512, 8, 2), (37, 16, 4), (5, 3, 1)):
        logits = g.standard_normal((T, E)).astype(np.float32)
        ids, w = P.moe_route(to_dev(logits), topk)
        ids_ref, w_ref = orc.moe_route(logits, topk)
        assert np.array_equal(ids.cpu().numpy(), ids_ref)
        assert np.allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)
    # ties go to the lower expert index
    ids, _ = P.moe_route(to_dev(np.zeros((4, 8), dtype=np.float32)), 2)
    assert ids.cpu().numpy().tolist() == [[0, 1]] * 4


@pytest.mark.parametrize("T,E,topk,bm", [(512, 8, 2, 64), (100, 8, 2, 16), (3000, 16, 4, 128),
                                         (7, 64, 2, 64), (300, 128, 4, 16), (600, 256, 8, 32)])
def test_align_matches_oracle(torch_cuda, orc, T, E, topk, bm):
    """Up to 64 experts the align kernel ranks pairs with a per-wave ballot table, above that
    expert by expert; both place every pair exactly as the oracle does (stable by pair)."""
    P = pkg()
    g = np.random.default_rng(71 + T)
    ids, _ = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    sorted_ids, expert_ids, npp = P.moe_align(to_dev(ids), E, bm)
    s_ref, e_ref, n_ref = orc.moe_align(ids, E, bm)
    n = int(npp.cpu().numpy()[0])
    assert n == n_ref
    assert np.array_equal(sorted_ids.cpu().numpy()[:n], s_ref)
    assert np.array_equal(expert_ids.cpu().numpy()[: n // bm], e_ref)
    assert np.all(sorted_ids.cpu().numpy()[n:] == T * topk)


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
@pytest.mark.parametrize("bm", [64, 128])
def test_grouped_gemm_matches_per_expert_dense(torch_cuda, orc, fmt, bm):
    """out[p] = a[p // topk] @ W16[expert of p] for every pair."""
    P = pkg()
    T, E, topk, K, N, G = 40, 4, 2, 256, 512, 128
    g = np.random.default_rng(72)
    x = synth.rand_x(g, T, K)
    ids, _ = orc.moe_route(g.standard_normal((T, E)).astype(np.float32), topk)
    qw, sc, qz = stacked_weights(fmt, E, K, N, G, 73)
    sorted_ids, expert_ids, npp = P.moe_align(to_dev(ids), E, bm)
    out = P.moe_gemm(to_dev(x), topk, to_dev(qw), to_dev(sc), to_dev(qz), sorted_ids, expert_ids,
                     npp, T * topk, N, K, fmt=FMT_NAME[fmt], group_size=G, block_m=bm)
    torch_cuda.cuda.synchronize()
    got = out.cpu().numpy()
    for e in range(E):
        pairs = np.nonzero(ids.ravel() == e)[0]
        if pairs.size == 0:
            continue
        ref = orc.w4a16_gemm(fmt, np.ascontiguousarray(x[pairs // topk]), qw[e], sc[e], qz[e], K, N,
                             G, want_f32=True)[1]
        assert_parity(got[pairs], ref, what=f"expert {e}")


def test_silu_mul_reference_entry_point(torch_cuda, orc):
    torch = torch_cuda
    P = pkg()
    g = np.random.default_rng(74)
    rows, inter = 33, 1024
    gu = (g.standard_normal((rows, 2 * inter)) * 3).astype(np.float16)
    out = torch.empty((rows, inter), dtype=torch.float16, device="cuda:0")
    P.fused_silu_mul_interleaved_f16(to_dev(gu), out, inter, rows * inter)
    got = out.cpu().numpy().astype(np.float64)
    ref = orc.silu_mul_f16(gu[:, :inter], gu[:, inter:]).reshape(rows, inter).astype(np.float64)
    # both round one f32 result to fp16; expf implementations may differ by an f32 ulp, which
    # moves the fp16 result by at most one fp16 ulp
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp + 1e-7)
    assert np.mean(got == ref) > 0.99


def test_moe_sum(torch_cuda):
    P = pkg()
    g = np.random.default_rng(75)
    T, topk, K = 64, 2, 512
    yp = g.standard_normal((T * topk, K)).astype(np.float16)
    w = g.random((T, topk)).astype(np.float32)
    y = P.moe_sum(to_dev(yp), to_dev(w), T, topk, K).cpu().numpy()
    ref = (yp.astype(np.float64).reshape(T, topk, K) * w[:, :, None]).sum(1)
    assert_parity(y, ref, tol=2e-3)


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
def test_fused_moe_small_vs_oracle(torch_cuda, orc, fmt):
    P = pkg()
    T, E, topk, K, I, G = 48, 4, 2, 256, 256, 128
    g = np.random.default_rng(76)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    w13 = stacked_weights(fmt, E, K, 2 * I, G, 77)
    w2 = stacked_weights(fmt, E, I, K, G, 78)
    y = P.fused_moe(to_dev(x), to_dev(logits), tuple(to_dev(a) for a in w13),
                    tuple(to_dev(a) for a in w2), topk=topk, fmt=FMT_NAME[fmt], group_size=G)
    torch_cuda.cuda.synchronize()
    ids, w = orc.moe_route(logits, topk)
    w13d = [orc.dequant(fmt, w13[0][e], w13[1][e], w13[2][e], K, 2 * I, G) for e in range(E)]
    w2d = [orc.dequant(fmt, w2[0][e], w2[1][e], w2[2][e], I, K, G) for e in range(E)]
    ref = orc.moe_forward(x, ids, w, w13d, w2d, inter=I)
    assert_parity(y.cpu().numpy(), ref.astype(np.float64), what="fused moe")


def test_fused_moe_config4_sampled_tokens(torch_cuda, orc):
    """Config 4 at full size (8 experts, top-2, T=512, K=4096, I=14336, GPTQ int4 G=128);
    the oracle recomputes 64 tokens through their experts: the first 16, the last 16 and
    32 drawn at random (about 30 s on 16 host threads)."""
    P = pkg()
    T, E, topk, K, I, G = 512, 8, 2, 4096, 14336, 128
    g = np.random.default_rng(0x5EED0004)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    w13 = stacked_weights(GPTQ, E, K, 2 * I, G, 0x5EED0104)
    w2 = stacked_weights(GPTQ, E, I, K, G, 0x5EED0204)
    y = P.fused_moe(to_dev(x), to_dev(logits), tuple(to_dev(a) for a in w13),
                    tuple(to_dev(a) for a in w2), topk=topk, fmt="gptq", group_size=G)
    y = y.cpu().numpy()
    assert np.all(np.isfinite(y))
    rest = np.random.default_rng(4).choice(np.arange(16, T - 16), 32, replace=False)
    toks = np.concatenate([np.arange(16), np.sort(rest), np.arange(T - 16, T)])
    ids, w = orc.moe_route(logits, topk)
    used = sorted(set(ids[toks].ravel().tolist()))
    dummy = np.zeros((8, 8), dtype=np.float16)
    w13d = [orc.dequant(GPTQ, w13[0][e], w13[1][e], w13[2][e], K, 2 * I, G) if e in used else dummy
            for e in range(E)]
    w2d = [orc.dequant(GPTQ, w2[0][e], w2[1][e], w2[2][e], I, K, G) if e in used else dummy
           for e in range(E)]
    ref = orc.moe_forward(np.ascontiguousarray(x[toks]), np.ascontiguousarray(ids[toks]),
                          np.ascontiguousarray(w[toks]), w13d, w2d, inter=I)
    assert_parity(y[toks], ref.astype(np.float64), what="config 4 sampled tokens")


def _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, fmt, G, g, what):
    """The oracle recomputes up to 5 sampled tokens (first, last, three random ones) of a
    fused layer through the dequantised weights of their experts."""
    host = lambda a: a.cpu().numpy() if hasattr(a, "cpu") else np.asarray(a)
    xs, ls = host(x), host(logits)
    T, K = xs.shape
    E = ls.shape[1]
    h13 = [None if a is None else host(a) for a in w13]
    h2 = [None if a is None else host(a) for a in w2]
    I = h2[1].shape[1] * G
    toks = np.unique(np.concatenate([[0, T - 1], g.integers(0, T, size=3)]))
    ids, w = orc.moe_route(ls, topk)
    used = set(ids[toks].ravel().tolist())
    dummy = np.zeros((8, 8), dtype=np.float16)
    w13d = [orc.dequant(fmt, h13[0][e], h13[1][e], None if h13[2] is None else h13[2][e], K, 2 * I, G)
            if e in used else dummy for e in range(E)]
    w2d = [orc.dequant(fmt, h2[0][e], h2[1][e], None if h2[2] is None else h2[2][e], I, K, G)
           if e in used else dummy for e in range(E)]
    ref = orc.moe_forward(np.ascontiguousarray(xs[toks]), np.ascontiguousarray(ids[toks]),
                          np.ascontiguousarray(w[toks]), w13d, w2d, inter=I)
    assert_parity(host(y)[toks], ref.astype(np.float64), what=f"{what}, tokens {toks.tolist()}")


def _layer_by_pieces(P, x, logits, w13, w2, topk, fmt, G, block_m):
    """The layer composed from the public pieces: route, align, grouped GEMM over block_m
    blocks, silu*mul, grouped GEMM, weighted sum."""
    import torch
    T, K = x.shape
    E = logits.shape[1]
    I = w2[1].shape[1] * G
    ids, w = P.moe_route(logits, topk)
    sorted_ids, expert_ids, npp = P.moe_align(ids, E, block_m)
    h = P.moe_gemm(x, topk, *w13, sorted_ids, expert_ids, npp, T * topk, 2 * I, K, fmt=fmt,
                   group_size=G, block_m=block_m)
    a = torch.empty((T * topk, I), dtype=torch.float16, device=x.device)
    P.fused_silu_mul_interleaved_f16(h, a, I, T * topk * I)
    yp = P.moe_gemm(a, 1, *w2, sorted_ids, expert_ids, npp, T * topk, K, I, fmt=fmt,
                    group_size=G, block_m=block_m)
    return P.moe_sum(yp, w, T, topk, K)


# The fused layer computes its grouped GEMMs over expert tiles (an expert's rows in one tile
# of 64/128/192/256 rows, 256/224/128 columns, chosen from the mean rows per expert and the CU
# count). Every pair row goes through the same arithmetic as in the block_m-block GEMM, so
# the layer must equal the composition of the public pieces bit for bit. Cases, with the
# tiles they take on a 256-CU MI355X: (T, E, topk, K, I, skew, fmt, block_m)
TILE_CASES = [
    (512, 8, 2, 256, 1792, None, GPTQ, 64),     # 192 x 224 (gate/up), 192 x 128 (down)
    (512, 8, 2, 256, 4096, None, AWQ, 128),     # 192 x 256, 192 x 128
    (512, 8, 2, 256, 256, 3, GPTQ, 64),         # expert 3 takes ~512 rows: 3 tiles of it
    (300, 8, 2, 512, 256, 0, AWQ, 64),          # 128-row tiles, expert 0 in 3 of them
    (1024, 4, 2, 256, 512, None, SYM, 128),     # 256-row tiles, two per expert
    (48, 4, 2, 256, 256, None, AWQ, 64),        # 64-row tiles
    (40, 64, 2, 256, 256, None, GPTQ, 64),      # 64-row tiles, most experts without tokens
]


@pytest.mark.parametrize("case", TILE_CASES, ids=[f"T{c[0]}_E{c[1]}_I{c[4]}_skew{c[5]}"
                                                  for c in TILE_CASES])
def test_fused_layer_expert_tiles_equal_block_composition(torch_cuda, orc, case):
    torch = torch_cuda
    T, E, topk, K, I, skew, fmt, bm = case
    P = pkg()
    g = np.random.default_rng(80 + T + I)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    if skew is not None:
        logits[:, skew] += 4.0          # nearly every token picks this expert
    G = 128
    w13 = tuple(to_dev(a) for a in stacked_weights(fmt, E, K, 2 * I, G, 81))
    w2 = tuple(to_dev(a) for a in stacked_weights(fmt, E, I, K, G, 82))
    if fmt == SYM:
        w13 = (w13[0], w13[1], None)
        w2 = (w2[0], w2[1], None)
    xd, ld = to_dev(x), to_dev(logits)
    y = P.fused_moe(xd, ld, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G, block_m=bm)
    ref = _layer_by_pieces(P, xd, ld, w13, w2, topk, FMT_NAME[fmt], G, 64)
    torch.cuda.synchronize()
    got, want = y.cpu().numpy().view(np.uint16), ref.cpu().numpy().view(np.uint16)
    diff = np.argwhere(got != want)
    assert diff.size == 0, f"{len(diff)} of {got.size} outputs differ, first at {diff[0].tolist()}"
    _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, fmt, G, g, f"tile case {case}")
    assert np.all(np.isfinite(y.cpu().numpy()))


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
def test_fused_layer_down_projection_split_k(torch_cuda, fmt):
    """A long down projection (I = 8192) splits its K over two workgroups per tile (fp32
    partials summed in split order): the layer stays within the GEMM tolerance of the
    block_m composition, and repeated calls are bit-identical."""
    T, E, topk, K, I, G = 512, 4, 2, 256, 8192, 128
    P = pkg()
    g = np.random.default_rng(90 + fmt)
    x = to_dev(synth.rand_x(g, T, K))
    logits = to_dev(g.standard_normal((T, E)).astype(np.float32))
    w13 = tuple(to_dev(a) for a in stacked_weights(fmt, E, K, 2 * I, G, 91))
    w2 = tuple(to_dev(a) for a in stacked_weights(fmt, E, I, K, G, 92))
    y1 = P.fused_moe(x, logits, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G)
    y2 = P.fused_moe(x, logits, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G)
    ref = _layer_by_pieces(P, x, logits, w13, w2, topk, FMT_NAME[fmt], G, 64)
    torch_cuda.cuda.synchronize()
    a, b = y1.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    assert np.all(np.isfinite(a))
    assert_parity(a, ref.cpu().numpy().astype(np.float64), what="split-K down projection")


def _moe_cases(n=10, seed=77):
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
def test_fused_layer_random_shapes_equal_block_composition(torch_cuda, orc, case):
    """Seeded random layers (token counts 1..700, 2..32 experts, top-1..4): the expert-tile
    layer equals the block_m composition of the pieces bit for bit, and the oracle recomputes
    up to 5 sampled tokens (first, last and three random ones) through their experts."""
    torch = torch_cuda
    T, E, topk, K, I, fmt = case
    P = pkg()
    g = np.random.default_rng(T * 31 + E * 7 + I)
    x = to_dev(synth.rand_x(g, T, K))
    logits = to_dev(g.standard_normal((T, E)).astype(np.float32))
    G = 128
    w13 = tuple(to_dev(a) for a in stacked_weights(fmt, E, K, 2 * I, G, 93))
    w2 = tuple(to_dev(a) for a in stacked_weights(fmt, E, I, K, G, 94))
    if fmt == SYM:
        w13, w2 = (w13[0], w13[1], None), (w2[0], w2[1], None)
    y = P.fused_moe(x, logits, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G)
    ref = _layer_by_pieces(P, x, logits, w13, w2, topk, FMT_NAME[fmt], G, 64)
    torch.cuda.synchronize()
    got, want = y.cpu().numpy().view(np.uint16), ref.cpu().numpy().view(np.uint16)
    diff = np.argwhere(got != want)
    assert diff.size == 0, f"{len(diff)} of {got.size} outputs differ, first at {diff[0].tolist()}"
    _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, fmt, G, g, f"random layer {case}")


# ------------------------------------------------- the layer on experts in the prepared layout

def _prepared_layer(P, xd, ld, w13, w2, topk, fmt, G, bm):
    w13p = P.prepare_layout_experts(*w13, fmt=FMT_NAME[fmt], group_size=G, zero_offset=1)
    w2p = P.prepare_layout_experts(*w2, fmt=FMT_NAME[fmt], group_size=G, zero_offset=1)
    return P.fused_moe_prepared(xd, ld, w13p, w2p, topk=topk, block_m=bm)


@pytest.mark.parametrize("case", TILE_CASES, ids=[f"T{c[0]}_E{c[1]}_I{c[4]}_skew{c[5]}"
                                                  for c in TILE_CASES])
def test_fused_moe_prepared_tile_cases(torch_cuda, orc, case):
    """w4a16_fused_moe_prepared over every expert-tile shape: within the GEMM tolerance of
    the layer on the checkpoint (the same weights W16, another order of the k sums within a
    stage), sampled tokens against the oracle, repeated calls bit-identical."""
    T, E, topk, K, I, skew, fmt, bm = case
    P = pkg()
    g = np.random.default_rng(180 + T + I)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    if skew is not None:
        logits[:, skew] += 4.0
    G = 128
    w13 = tuple(to_dev(a) for a in stacked_weights(fmt, E, K, 2 * I, G, 181))
    w2 = tuple(to_dev(a) for a in stacked_weights(fmt, E, I, K, G, 182))
    if fmt == SYM:
        w13 = (w13[0], w13[1], None)
        w2 = (w2[0], w2[1], None)
    xd, ld = to_dev(x), to_dev(logits)
    y = _prepared_layer(P, xd, ld, w13, w2, topk, fmt, G, bm)
    y2 = _prepared_layer(P, xd, ld, w13, w2, topk, fmt, G, bm)
    ck = P.fused_moe(xd, ld, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G, block_m=bm)
    torch_cuda.cuda.synchronize()
    a = y.cpu().numpy()
    assert np.array_equal(a.view(np.uint16), y2.cpu().numpy().view(np.uint16))
    assert np.all(np.isfinite(a))
    assert_parity(a, ck.cpu().numpy().astype(np.float64), what=f"prepared vs checkpoint {case}")
    _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, fmt, G, g, f"prepared tile case {case}")


@pytest.mark.parametrize("fmt", [GPTQ, AWQ])
def test_fused_moe_prepared_down_projection_split_k(torch_cuda, orc, fmt):
    """I = 8192: the prepared down projection splits its K over two workgroups per tile."""
    T, E, topk, K, I, G = 512, 4, 2, 256, 8192, 128
    P = pkg()
    g = np.random.default_rng(190 + fmt)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    w13 = tuple(to_dev(a) for a in stacked_weights(fmt, E, K, 2 * I, G, 191))
    w2 = tuple(to_dev(a) for a in stacked_weights(fmt, E, I, K, G, 192))
    xd, ld = to_dev(x), to_dev(logits)
    y = _prepared_layer(P, xd, ld, w13, w2, topk, fmt, G, 64)
    ck = P.fused_moe(xd, ld, w13, w2, topk=topk, fmt=FMT_NAME[fmt], group_size=G)
    torch_cuda.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ck.cpu().numpy().astype(np.float64), what="prepared split-K down")
    _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, fmt, G, g, "prepared split-K down")


def test_fused_moe_prepared_config4(torch_cuda, orc):
    """Config 4 at full size on prepared experts: every token within the GEMM tolerance of
    the layer on the checkpoint, sampled tokens against the oracle."""
    P = pkg()
    T, E, topk, K, I, G = 512, 8, 2, 4096, 14336, 128
    g = np.random.default_rng(0x5EED0004)
    x = synth.rand_x(g, T, K)
    logits = g.standard_normal((T, E)).astype(np.float32)
    w13 = tuple(to_dev(a) for a in stacked_weights(GPTQ, E, K, 2 * I, G, 0x5EED0104))
    w2 = tuple(to_dev(a) for a in stacked_weights(GPTQ, E, I, K, G, 0x5EED0204))
    xd, ld = to_dev(x), to_dev(logits)
    ck = P.fused_moe(xd, ld, w13, w2, topk=topk, fmt="gptq", group_size=G).cpu().numpy()
    y = _prepared_layer(P, xd, ld, w13, w2, topk, GPTQ, G, 64)
    torch_cuda.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ck.astype(np.float64), what="config 4 prepared vs checkpoint")
    _check_sampled_tokens(orc, y, x, logits, w13, w2, topk, GPTQ, G, g, "config 4 prepared")


def test_fused_moe_prepared_rejects_unsupported_groups(torch_cuda):
    """Group size 32 has a prepared layout but no expert-tile B stage: Unsupported."""
    P = pkg()
    T, E, topk, K, I, G = 32, 4, 2, 256, 256, 32
    g = np.random.default_rng(199)
    w13 = tuple(to_dev(a) for a in stacked_weights(GPTQ, E, K, 2 * I, G, 198))
    w2 = tuple(to_dev(a) for a in stacked_weights(GPTQ, E, I, K, G, 197))
    w13p = P.prepare_layout_experts(*w13, fmt="gptq", group_size=G)
    w2p = P.prepare_layout_experts(*w2, fmt="gptq", group_size=G)
    with pytest.raises(P.Unsupported):
        P.fused_moe_prepared(to_dev(synth.rand_x(g, T, K)), to_dev(g.standard_normal((T, E)).astype(np.float32)),
                             w13p, w2p, topk=topk)
