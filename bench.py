"""Benchmark of the MI355X W4A16 path (one JSON line on stdout).

Headline (the metric's M=1 case, config 1): AWQ int4 GEMV, M=1, K=4096 -> N=14336, G=128,
weights rotated over enough distinct buffers (> 512 MB) that the 256 MB Infinity Cache
cannot hold them. The weights are given as AWQ checkpoints and rewritten once each into the
prepared layout (w4a16_prepare_layout: the load-time step, timed on its own and reported);
one step = one w4a16_gemm_prepared call through the C ABI. The same workload on the
checkpoint layout as stored (w4a16_gemm) is reported beside it in extra.checkpoint_layout. The timed region is
exactly --steps calls, with untimed calls (HIP graph replays) enqueued just ahead of the start
event so that the GPU is busy while the host enqueues the timed work: up to DIRECT_MAX_STEPS
steps are launched directly behind about 1000 such calls (a graph replay has a fixed cost of
its own, ~8 us, that a short region would carry), more steps are replayed from HIP graphs so
that host launch cost does not gate the GPU. `value` is algorithmic GB/s (bytes of qweight + scales +
qzeros + x + out, each counted once) over that region, measured with HIP events on the
launch stream; the median of five further batches of 1000 calls is reported beside it.
(Act-order lines in "extra" also count the int32 g_idx, or the prepared path's permutation.)

roofline.traffic: HBM bytes per launch of the headline kernel from two rocprofv3 --pmc
passes (FETCH_SIZE, then WRITE_SIZE) over a child run of this script (--pmc-child), each
divided by the ratio that the same counter reads for a plain streaming kernel of known
size (torch's neg over 512 MiB of int32) in the same child run.

Secondary figures (same line, "extra"): AWQ prefill M=2048 in both MLP shapes (TFLOP/s,
2*M*N*K), the other decode/small-batch shapes, one GPU's share of an 8-way tensor-parallel
MLP (tp8_*), and the fused MoE layer of config 4.
cpu_baseline: the CPU oracle (dequant + fp32-accumulate matmul, OpenMP) on a bounded
sample of the same workload, timed on this host's cores.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import platform
import shutil
import subprocess
import sys
import tempfile
import time
import zlib

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_DENSE_PEAK_TFLOPS = 2516.6  # MI355X fp16 dense MFMA
GRAPH_CALLS = 100
# the headline's timed region up to this many steps is launched directly (behind ~1000 untimed
# graph-replayed calls) instead of as graph replays: one replay of a 20-call graph took 144 us
# against 20 x 6.78 us for the same calls inside longer graphs (~8.5 us per replay), direct
# launches 7.03 us per call
DIRECT_MAX_STEPS = 100
PMC_WARM, PMC_MEASURED = 20, 40
COPY_ELEMS = 128 * 1024 * 1024   # int32 elements streamed by the calibration kernel (512 MiB)

HEADLINE = ("awq", 1, 4096, 14336, 128)


def algorithmic_bytes(fmt: str, M: int, K: int, N: int, G: int, act_order: bool = False) -> int:
    """Bytes a call must move, each tensor counted once: qweight, scales, qzeros (none for
    the symmetric format), the int32 g_idx (or the prepared path's permutation) for
    act-order, x and out."""
    qweight = K * N // 2
    scales = (K // G) * N * 2
    qzeros = 0 if fmt == "gptq_sym" else (K // G) * N // 2
    gidx = K * 4 if act_order else 0
    return qweight + scales + qzeros + gidx + M * K * 2 + M * N * 2


def make_weight_sets(torch, fmt, K, N, G, count, dev, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    sets = []
    shape_qw = (K, N // 8) if fmt == "awq" else (K // 8, N)
    for _ in range(count):
        qw = torch.randint(-2 ** 31, 2 ** 31 - 1, shape_qw, dtype=torch.int32, device=dev, generator=gen)
        qz = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // G, N // 8), dtype=torch.int32, device=dev,
                           generator=gen)
        sc = (torch.rand((K // G, N), device=dev, generator=gen) * 0.018 + 0.002).half()
        sets.append((qw, sc, qz))
    torch.cuda.synchronize()   # generated on the default stream; the calls run on another
    return sets


def _capture(torch, fn, n_calls, n_graphs, stream):
    """n_graphs HIP graphs of n_calls calls each; fn(i) enqueues call i on the current stream."""
    graphs = []
    for gi in range(n_graphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for j in range(n_calls):
                fn(gi * n_calls + j)
        graphs.append(g)
    return graphs


def _timed_replays(torch, graphs, reps, stream, lead=None):
    """ms for `reps` graph replays. Untimed replays (`lead`, default the last of `graphs`) are
    enqueued right before the start event (no synchronisation in between), so the GPU is still
    busy with them while the host enqueues the timed replays: host launch latency stays out of
    the timed region."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for g in (lead if lead else graphs[-1:]):
            g.replay()
        start.record(stream)
        for r in range(reps):
            graphs[r % len(graphs)].replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def _timed_direct(torch, fn, steps, stream, lead):
    """ms for `steps` direct calls fn(0 .. steps-1), enqueued behind the untimed graph replays
    `lead` (no synchronisation in between), which keep the GPU busy while the host enqueues
    the timed calls."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for g in lead:
            g.replay()
        start.record(stream)
        for i in range(steps):
            fn(i)
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def time_calls(torch, fn, steps, warmup, stream, n_sets, batches=5, batch_calls=1000,
               graph_calls=GRAPH_CALLS, n_graphs=10, exact_direct=False):
    """Per-call ms of fn(i) (call i uses weight set i % n_sets) replayed from HIP graphs.

    Returns (ms_exact, ms_median, batch_ms, wall_s): ms_exact from exactly `steps` calls
    (with exact_direct and at most DIRECT_MAX_STEPS steps: launched directly behind the batch
    graphs' replays; else graphs of C = the largest divisor of steps up to graph_calls calls),
    ms_median the median over `batches` further batches of about `batch_calls` calls (graphs
    of graph_calls)."""
    with torch.cuda.stream(stream):
        for i in range(max(warmup, n_sets)):
            fn(i)
    stream.synchronize()
    direct = exact_direct and steps <= DIRECT_MAX_STEPS
    c = max(d for d in range(1, min(graph_calls, steps) + 1) if steps % d == 0)
    g_exact = [] if direct else _capture(torch, fn, c, max(1, min(steps // c, n_graphs)), stream)
    g_batch = g_exact if c == graph_calls and not direct else _capture(torch, fn, graph_calls, n_graphs, stream)
    with torch.cuda.stream(stream):
        for g in g_exact + g_batch:
            g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if direct:
        ms_exact = _timed_direct(torch, fn, steps, stream, lead=g_batch) / steps
    else:
        # a short graph-timed region is preceded by the batch graphs, about 1000 calls of
        # other graph instances (a relaunch of an instance still in flight is not queued
        # behind it), so the host has enqueued it before the GPU gets there
        lead = g_batch if g_batch is not g_exact else None
        ms_exact = _timed_replays(torch, g_exact, steps // c, stream, lead=lead) / steps
    wall = time.perf_counter() - t0
    reps = max(1, batch_calls // graph_calls)
    per = []
    for _ in range(batches):
        per.append(_timed_replays(torch, g_batch, reps, stream) / (reps * graph_calls))
    per.sort()
    return ms_exact, per[len(per) // 2], per, wall


def time_graphs(torch, pkg, x, sets, out, fmt, G, steps, warmup, stream, g_idx=None):
    """Median per-call ms of w4a16_gemm over rotated weight sets (5 batches of `steps` calls)."""
    n = len(sets)

    def fn(i):
        qw, sc, qz = sets[i % n]
        pkg.gemm(x, qw, sc, qz, fmt=fmt, group_size=G, g_idx=g_idx, out=out)
    return time_calls(torch, fn, GRAPH_CALLS, warmup, stream, n, batch_calls=max(steps, GRAPH_CALLS))[1]


def time_direct(torch, fn, calls, stream, warm=3):
    """Average ms of fn() launched `calls` times on `stream` (HIP events on that stream)."""
    with torch.cuda.stream(stream):
        for i in range(warm):
            fn(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(calls):
            fn(i)
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / calls


def cpu_baseline(fmt_id, x, qw, sc, qz, M, K, N, G, budget_s=15.0):
    """CPU oracle (test infrastructure) timed on a bounded sample: whole calls of the same
    workload (dequant + fp32-accumulate matmul), repeated until ~budget_s of work (1 warm-up
    excluded), then the dequantisation alone for a third of that budget. Medians."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    def med_of(fn, budget):
        fn()   # warm-up
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= 200:
                break
        times.sort()
        return times[len(times) // 2], len(times)

    med, n = med_of(lambda: oracle.w4a16_gemm(fmt_id, x, qw, sc, qz, K, N, G, acc64=False), budget_s)
    med_dq, n_dq = med_of(lambda: oracle.dequant(fmt_id, qw, sc, qz, K, N, G), budget_s / 3)
    return med, n, med_dq, n_dq, oracle.num_threads()


def progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# ----------------------------------------------------------------------------- traffic

# Workloads a counter run (--pmc-child) can drive, (fmt, M, K, N, G, act_order) each: the
# configs at the sizes the metric names. "c4_moe" is config 4's fused MoE layer.
PMC_WORKLOADS = {
    "headline": HEADLINE + (False,),
    "c0": ("gptq_sym", 1, 4096, 4096, 128, False),
    "c1_m1_k14336_n4096": ("awq", 1, 14336, 4096, 128, False),
    "c1_m4_k4096_n14336": ("awq", 4, 4096, 14336, 128, False),
    "c1_m4_k14336_n4096": ("awq", 4, 14336, 4096, 128, False),
    "c1_m8_k4096_n14336": ("awq", 8, 4096, 14336, 128, False),
    "c1_m8_k14336_n4096": ("awq", 8, 14336, 4096, 128, False),
    "c2_m16": ("gptq", 16, 4096, 6144, 128, True),
    "c2_m32": ("gptq", 32, 4096, 6144, 128, True),
    "c2_m64": ("gptq", 64, 4096, 6144, 128, True),
    "c2_plain_m16": ("gptq", 16, 4096, 6144, 128, False),
    "c2_plain_m32": ("gptq", 32, 4096, 6144, 128, False),
    "c2_plain_m64": ("gptq", 64, 4096, 6144, 128, False),
    "c3_k4096_n14336": ("awq", 2048, 4096, 14336, 128, False),
    "c3_k14336_n4096": ("awq", 2048, 14336, 4096, 128, False),
    "c4_moe": None,
    # the same shapes on weights in the prepared layout (w4a16_prepare_layout)
    "prep_headline": HEADLINE + (False,),
    "prep_c0": ("gptq_sym", 1, 4096, 4096, 128, False),
    "prep_c1_m1_k14336_n4096": ("awq", 1, 14336, 4096, 128, False),
    "prep_c1_m8_k4096_n14336": ("awq", 8, 4096, 14336, 128, False),
    "prep_c3_k4096_n14336": ("awq", 2048, 4096, 14336, 128, False),
    "prep_c3_k14336_n4096": ("awq", 2048, 14336, 4096, 128, False),
    # the prepared small-batch kernel (x rewritten in fragment order first), plain and
    # act-order (group-order repack, then the layout; x gathered by perm per call)
    "prep_c2_plain_m16": ("gptq", 16, 4096, 6144, 128, False),
    "prep_c2_plain_m64": ("gptq", 64, 4096, 6144, 128, False),
    "prep_c2_m16": ("gptq", 16, 4096, 6144, 128, True),
    "prep_c2_m64": ("gptq", 64, 4096, 6144, 128, True),
    # act-order beyond 64 rows through w4a16_gemm: 128 rows (small-batch kernel in two row
    # chunks) and 2048 (group order computed per call, then the prefill kernel)
    "c2_m128": ("gptq", 128, 4096, 6144, 128, True),
    "c2_m2048": ("gptq", 2048, 4096, 6144, 128, True),
    # act-order on the prepared layout of the checkpoint as stored, g_idx per row
    # (w4a16_gemm_prepared_gidx)
    "prepstored_c2_m16": ("gptq", 16, 4096, 6144, 128, True),
    "prepstored_c2_m32": ("gptq", 32, 4096, 6144, 128, True),
    "prepstored_c2_m64": ("gptq", 64, 4096, 6144, 128, True),
}


def c2_g_idx(torch, dev, K=4096, G=128):
    """Config 2's act-order groups: a seeded random permutation of repeat(0..K/G-1, G)."""
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(2))
    return (torch.arange(K) // G)[perm].to(torch.int32).to(dev)


def moe_layer(torch, dev, gen):
    """Config 4's layer: T=512 tokens, 8 experts, top-2, K=4096, I=14336, GPTQ G=128, random
    packed words, scales in [0.002, 0.02], fp32 router logits ~ N(0, 1)."""
    T, E, topk, K, I, G = 512, 8, 2, 4096, 14336, 128

    def words(*shape):
        return torch.randint(-2 ** 31, 2 ** 31 - 1, shape, dtype=torch.int32, device=dev, generator=gen)

    def scales(*shape):
        return (torch.rand(shape, device=dev, generator=gen) * 0.018 + 0.002).half()

    w13 = (words(E, K // 8, 2 * I), scales(E, K // G, 2 * I), words(E, K // G, 2 * I // 8))
    w2 = (words(E, I // 8, K), scales(E, I // G, K), words(E, I // G, K // 8))
    x = torch.randn((T, K), device=dev, generator=gen).half()
    logits = torch.randn((T, E), device=dev, generator=gen)
    return {"T": T, "E": E, "topk": topk, "K": K, "I": I, "G": G, "w13": w13, "w2": w2,
            "x": x, "logits": logits}


def pmc_child(args) -> int:
    """Workload profiled by the counter passes: PMC_WARM + PMC_MEASURED launches of the chosen
    workload (--pmc-workload; the headline by default) over rotated weight sets, then three
    launches of the calibration kernel."""
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    if args.pmc_workload == "c4_moe":
        gen = torch.Generator(device=dev)
        gen.manual_seed(0x5EED0004)
        L = moe_layer(torch, dev, gen)
        out = torch.empty((L["T"], L["K"]), dtype=torch.float16, device=dev)
        for _ in range(PMC_WARM + PMC_MEASURED):
            pkg.fused_moe(L["x"], L["logits"], L["w13"], L["w2"], topk=L["topk"], out=out)
        del L
    else:
        fmt, M, K, N, G, act_order = PMC_WORKLOADS[args.pmc_workload]
        n_sets = args.sets if M <= 64 else 2
        sets = make_weight_sets(torch, fmt, K, N, G, n_sets, dev, seed=0x5EED0001)
        g_idx = c2_g_idx(torch, dev, K, G) if act_order else None
        x = torch.randn((M, K), device=dev).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        if args.pmc_workload.startswith("prepstored_"):
            prep = [pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G, zero_offset=1)
                    for qw, sc, qz in sets]
            del sets
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            for i in range(PMC_WARM + PMC_MEASURED):
                pkg.gemm_prepared(x, prep[i % len(prep)], g_idx=g_idx, out=out)
            sets = prep
        elif args.pmc_workload.startswith("prep_"):
            perm = None
            if act_order:   # group order once, then the layout of the repacked rows
                prep = []
                for qw, sc, qz in sets:
                    qs, perm = pkg.prepare_act_order(qw, g_idx, group_size=G)
                    prep.append(pkg.prepare_layout(qs, sc, qz, fmt=fmt, group_size=G, zero_offset=1))
            else:
                prep = [pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G, zero_offset=1)
                        for qw, sc, qz in sets]
            del sets
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            for i in range(PMC_WARM + PMC_MEASURED):
                pkg.gemm_prepared(x, prep[i % len(prep)], perm=perm, out=out)
            sets = prep
        else:
            for i in range(PMC_WARM + PMC_MEASURED):
                pkg.gemm(x, *sets[i % len(sets)], fmt=fmt, group_size=G, g_idx=g_idx, out=out)
        del sets
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    src = torch.ones(COPY_ELEMS, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("pmc child done", flush=True)
    return 0


def _counter_table(csv_dir):
    """{kernel name: {counter: [value per dispatch, in dispatch order]}} of a counter run."""
    files = glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True)
    rows = {}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                rows.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], []).append(
                    (int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    return {k: {c: [v for _, v in sorted(vals)] for c, vals in cs.items()} for k, cs in rows.items()}


def _counter_means(csv_dir, counter):
    """Per-dispatch mean of `counter` for the library's kernel (last PMC_MEASURED dispatches)
    and for the calibration kernel."""
    table = _counter_table(csv_dir)
    ours = [v for k, cs in table.items() if "w4a16::" in k for v in cs.get(counter, [])]
    copy = [v for k, cs in table.items() if "neg_kernel" in k for v in cs.get(counter, [])]
    ours = ours[-PMC_MEASURED:]
    if not ours or not copy:
        raise RuntimeError(f"{counter}: no samples (ours {len(ours)}, copy {len(copy)})")
    return sum(ours) / len(ours), sum(copy) / len(copy)


def _rocprof_pass(rocprof, counters, workload, sets, outdir):
    """One rocprofv3 --pmc run of a --pmc-child process; returns its counter table."""
    env = dict(os.environ, TMPDIR="/tmp")
    d = os.path.join(outdir, "_".join(counters)[:80])
    cmd = ["timeout", "-s", "KILL", "120", rocprof, "--pmc", *counters, "--output-format", "csv",
           "-d", d, "-o", "pmc", "--", sys.executable, os.path.abspath(__file__),
           "--pmc-child", "--pmc-workload", workload, "--sets", str(sets)]
    r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
    if r.returncode != 0:
        tail = (r.stdout + r.stderr).strip().splitlines()[-3:]
        raise RuntimeError(f"{counters} pass failed rc={r.returncode}: {tail}")
    return _counter_table(d)


def pmc_report(args) -> int:
    """Counter report of one workload (--pmc-workload), one JSON line. Default passes:
    FETCH_SIZE, then WRITE_SIZE, each calibrated against the copy kernel of the same run, per
    library kernel: HBM bytes per dispatch beside the algorithmic bytes. With --pmc-counters
    (one pass per ';'-separated group of space-separated counters): the per-dispatch means
    of those counters per library kernel. Means are over each kernel's last PMC_MEASURED
    dispatches."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    outdir = tempfile.mkdtemp(prefix="w4a16_pmc_", dir="/tmp")
    groups = ([g.split() for g in args.pmc_counters.split(";") if g.strip()]
              if args.pmc_counters else [["FETCH_SIZE"], ["WRITE_SIZE"]])
    rep = {"workload": args.pmc_workload, "passes": [], "measured_dispatches": PMC_MEASURED}
    spec = PMC_WORKLOADS[args.pmc_workload]
    if spec is not None:
        fmt, M, K, N, G, act_order = spec
        rep["algorithmic_bytes"] = algorithmic_bytes(fmt, M, K, N, G, act_order)
    traffic = {}
    for counters in groups:
        table = _rocprof_pass(rocprof, counters, args.pmc_workload, args.sets, outdir)
        kern = {}
        for name, cs in table.items():
            if "w4a16" not in name:   # demangled or mangled (_ZN5w4a16...) names
                continue
            kern[name] = {c: round(sum(v[-PMC_MEASURED:]) / len(v[-PMC_MEASURED:]), 1)
                          for c, v in cs.items()}
            kern[name]["dispatches"] = max(len(v) for v in cs.values())
        entry = {"counters": counters, "kernels": kern}
        copy = [v for k, cs in table.items() if "neg_kernel" in k for c, vals in cs.items()
                for v in vals if c in ("FETCH_SIZE", "WRITE_SIZE")]
        if copy and counters in (["FETCH_SIZE"], ["WRITE_SIZE"]):
            factor = (sum(copy) / len(copy)) * 1024.0 / (COPY_ELEMS * 4)
            entry["calibration_factor"] = round(factor, 4)
            for name, cs in kern.items():
                traffic[name] = traffic.get(name, 0.0) + cs[counters[0]] * 1024.0 / factor
        rep["passes"].append(entry)
    shutil.rmtree(outdir, ignore_errors=True)
    if traffic:
        rep["traffic_bytes_per_dispatch"] = {k: int(v) for k, v in traffic.items()}
        if "algorithmic_bytes" in rep:
            rep["traffic_over_algorithmic"] = {
                k: round(v / rep["algorithmic_bytes"], 3) for k, v in traffic.items()}
    print(json.dumps(rep), flush=True)
    return 0


def measure_traffic(args):
    """HBM bytes per headline launch from two rocprofv3 --pmc passes, calibrated."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rocprof):
        return None, {"traffic_note": "rocprofv3 not found"}
    env = dict(os.environ, TMPDIR="/tmp")
    outdir = tempfile.mkdtemp(prefix="w4a16_pmc_", dir="/tmp")
    detail = {}
    copy_bytes = COPY_ELEMS * 4
    total = 0.0
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(outdir, counter)
        cmd = ["timeout", "-s", "KILL", "90", rocprof, "--pmc", counter, "--output-format", "csv",
               "-d", d, "-o", "pmc", "--", sys.executable, os.path.abspath(__file__),
               "--pmc-child", "--pmc-workload", "prep_headline", "--sets", str(args.sets)]
        r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
        if r.returncode != 0:
            tail = (r.stdout + r.stderr).strip().splitlines()[-3:]
            return None, {"traffic_note": f"{counter} pass failed rc={r.returncode}: {tail}"}
        ours_kib, copy_kib = _counter_means(d, counter)
        factor = copy_kib * 1024.0 / copy_bytes
        total += ours_kib * 1024.0 / factor
        detail[counter] = {"headline_KiB_per_dispatch": round(ours_kib, 1),
                           "copy_KiB_per_dispatch": round(copy_kib, 1),
                           "calibration_factor": round(factor, 4)}
    shutil.rmtree(outdir, ignore_errors=True)
    return int(total), {"traffic_counters": detail,
                        "traffic_calibration": f"torch.neg over {copy_bytes >> 20} MiB int32 "
                                               f"(reads and writes {copy_bytes >> 20} MiB)"}


# ----------------------------------------------------------------------------- extras

def extras(torch, pkg, dev, stream, args):
    """Secondary shapes: the other configs at the sizes the metric names, the prepared
    act-order path, the reference-named typed entry points, and achievable references."""
    res = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x5EED0003)

    def record(tag, fmt, M, K, N, G, ms, kernel, act_order=False):
        nbytes = algorithmic_bytes(fmt, M, K, N, G, act_order)
        tfl = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        res[tag] = {"kernel": kernel, "us_per_call": round(ms * 1e3, 2),
                    "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "TFLOPs": round(tfl, 2),
                    "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "frac_mfma": round(tfl / FP16_DENSE_PEAK_TFLOPS, 4)}
        progress(f"{tag}: {res[tag]['us_per_call']} us")

    def gemm_case(tag, fmt, M, K, N, G, n_sets, calls, g_idx=None, bf16=False):
        sets = make_weight_sets(torch, fmt, K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        dt = torch.bfloat16 if bf16 else torch.float16
        if bf16:   # activations, scales and output in bfloat16 (W4A16_BF16)
            sets = [(qw, sc.to(dt), qz) for qw, sc, qz in sets]
        x = torch.randn((M, K), device=dev, generator=gen).to(dt)
        out = torch.empty((M, N), dtype=dt, device=dev)
        # graph replays for every size: steady-state clocks, no host launch gaps
        ms = time_graphs(torch, pkg, x, sets, out, fmt, G, calls, 10, stream, g_idx=g_idx)
        record(tag, fmt, M, K, N, G, ms, pkg.plan(fmt, M, N, K, G, has_g_idx=g_idx is not None, bf16=bf16),
               act_order=g_idx is not None)
        del sets

    gemm_case("c0_gptq_sym_m1_k4096_n4096", "gptq_sym", 1, 4096, 4096, 128, 60, 1000)
    for M in (4, 8):
        gemm_case(f"c1_awq_m{M}_k4096_n14336", "awq", M, 4096, 14336, 128, 20, 1000)
    for M in (1, 4, 8):
        gemm_case(f"c1_awq_m{M}_k14336_n4096", "awq", M, 14336, 4096, 128, 20, 1000)
    g_idx = c2_g_idx(torch, dev)
    # 40 weight sets of 13.4 MB (537 MB, past the 256 MB Infinity Cache)
    for M in (16, 32, 64):
        gemm_case(f"c2_gptq_actorder_m{M}_k4096_n6144", "gptq", M, 4096, 6144, 128, 40, 500,
                  g_idx=g_idx)
        gemm_case(f"c2_gptq_m{M}_k4096_n6144_no_gidx", "gptq", M, 4096, 6144, 128, 40, 500)
    # the same act-order weights at prefill size through w4a16_gemm (group order computed on the
    # device per call, rows repacked, x gathered, then the prefill kernel)
    gemm_case("c2_gptq_actorder_m2048_k4096_n6144", "gptq", 2048, 4096, 6144, 128, 2, 200, g_idx=g_idx)
    gemm_case("c2_gptq_m2048_k4096_n6144_no_gidx", "gptq", 2048, 4096, 6144, 128, 2, 200)
    # between the two: 128 rows (act-order: the small-batch kernel in two row chunks)
    gemm_case("c2_gptq_actorder_m128_k4096_n6144", "gptq", 128, 4096, 6144, 128, 8, 300, g_idx=g_idx)
    gemm_case("c2_gptq_m128_k4096_n6144_no_gidx", "gptq", 128, 4096, 6144, 128, 8, 300)

    # config 2's act-order layer through the one-time group-order repack: gather + plain kernel
    def prepared_case(tag, M, n_sets, calls):
        K, N, G = 4096, 6144, 128
        sets = make_weight_sets(torch, "gptq", K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        prep = [pkg.prepare_act_order(qw, g_idx, group_size=G) for qw, _, _ in sets]
        x = torch.randn((M, K), device=dev, generator=gen).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)

        def fn(i):
            qp, pm = prep[i % n_sets]
            _, sc, qz = sets[i % n_sets]
            pkg.gemm_act_order(x, qp, sc, qz, pm, group_size=G, out=out)
        ms = time_calls(torch, fn, GRAPH_CALLS, 10, stream, n_sets, batch_calls=calls,
                        n_graphs=min(10, max(1, 1000 // GRAPH_CALLS)))[1]
        record(tag, "gptq", M, K, N, G, ms, "gather+" + pkg.plan("gptq", M, N, K, G),
               act_order=True)
        del sets, prep

    for M in (16, 64):
        prepared_case(f"c2_gptq_actorder_prepared_m{M}_k4096_n6144", M, 40, 500)
    prepared_case("c2_gptq_actorder_prepared_m2048_k4096_n6144", 2048, 2, 200)

    # config 2's act-order layer in the prepared layout (group-order repack, then
    # w4a16_prepare_layout, once): per call, x gathered by perm straight into the small-batch
    # kernel's operand order, then the small-batch kernel (prefill kernel at M = 2048)
    def preplayout_case(tag, M, n_sets, calls):
        K, N, G = 4096, 6144, 128
        sets = make_weight_sets(torch, "gptq", K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        preps = []
        for qw, sc, qz in sets:
            qp, pm = pkg.prepare_act_order(qw, g_idx, group_size=G)
            preps.append((pkg.prepare_layout(qp, sc, qz, fmt="gptq", group_size=G, zero_offset=1), pm))
        del sets
        x = torch.randn((M, K), device=dev, generator=gen).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)

        def fn(i):
            w, pm = preps[i % n_sets]
            pkg.gemm_prepared(x, w, perm=pm, out=out)
        ms = time_calls(torch, fn, GRAPH_CALLS, 10, stream, n_sets, batch_calls=calls,
                        n_graphs=min(10, max(1, 1000 // GRAPH_CALLS)))[1]
        record(tag, "gptq", M, K, N, G, ms, "gather+prepared/" + ("prefill" if M > 64 else "small-batch"),
               act_order=True)
        del preps

    for M in (16, 32, 64):
        preplayout_case(f"c2_gptq_actorder_preplayout_m{M}_k4096_n6144", M, 40, 500)
    preplayout_case("c2_gptq_actorder_preplayout_m2048_k4096_n6144", 2048, 2, 200)

    # config 2's act-order layer prepared as stored (w4a16_prepare_layout on the checkpoint, rows
    # in their own order): per call, w4a16_gemm_prepared_gidx with g_idx (no repack, no gather)
    def prepstored_case(tag, M, n_sets, calls):
        K, N, G = 4096, 6144, 128
        sets = make_weight_sets(torch, "gptq", K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        preps = [pkg.prepare_layout(qw, sc, qz, fmt="gptq", group_size=G, zero_offset=1)
                 for qw, sc, qz in sets]
        del sets
        x = torch.randn((M, K), device=dev, generator=gen).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)

        def fn(i):
            pkg.gemm_prepared(x, preps[i % n_sets], g_idx=g_idx, out=out)
        ms = time_calls(torch, fn, GRAPH_CALLS, 10, stream, n_sets, batch_calls=calls,
                        n_graphs=min(10, max(1, 1000 // GRAPH_CALLS)))[1]
        record(tag, "gptq", M, K, N, G, ms, "prepared+g_idx/small-batch", act_order=True)
        del preps

    for M in (16, 32, 64):
        prepstored_case(f"c2_gptq_actorder_prepstored_m{M}_k4096_n6144", M, 40, 500)

    gemm_case("c3_awq_m2048_k4096_n14336", "awq", 2048, 4096, 14336, 128, 2, 300)
    gemm_case("c3_awq_m2048_k14336_n4096", "awq", 2048, 14336, 4096, 128, 2, 300)
    # the same workloads with bfloat16 activations, scales and output
    gemm_case("bf16_c0_gptq_sym_m1_k4096_n4096", "gptq_sym", 1, 4096, 4096, 128, 60, 1000, bf16=True)
    for M in (1, 8):
        gemm_case(f"bf16_c1_awq_m{M}_k4096_n14336", "awq", M, 4096, 14336, 128, 20, 1000, bf16=True)
    gemm_case("bf16_c2_gptq_m16_k4096_n6144_no_gidx", "gptq", 16, 4096, 6144, 128, 40, 500, bf16=True)
    gemm_case("bf16_c3_awq_m2048_k4096_n14336", "awq", 2048, 4096, 14336, 128, 2, 300, bf16=True)

    # the prepared layout (w4a16_prepare_layout once per weight set, then w4a16_gemm_prepared);
    # the one-time prepare is timed on its own (one call, after a warm-up call)
    def layout_case(tag, fmt, M, K, N, G, n_sets, calls):
        sets = make_weight_sets(torch, fmt, K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        qw, sc, qz = sets[0]
        pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G, zero_offset=1)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G, zero_offset=1)
        ev1.record()
        torch.cuda.synchronize()
        prep_us = ev0.elapsed_time(ev1) * 1e3
        preps = []
        for i in range(n_sets):
            qw, sc, qz = sets[i]
            preps.append(pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G, zero_offset=1))
            sets[i] = None   # the checkpoint copy is not needed any more
        torch.cuda.synchronize()
        del sets
        torch.cuda.empty_cache()
        x = torch.randn((M, K), device=dev, generator=gen).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)

        def fn(i):
            pkg.gemm_prepared(x, preps[i % n_sets], out=out)
        ms = time_calls(torch, fn, GRAPH_CALLS, 10, stream, n_sets, batch_calls=calls)[1]
        record(tag, fmt, M, K, N, G, ms, "prepared/" + ("gemv" if M <= 8 else "prefill"))
        res[tag]["prepare_once_us"] = round(prep_us, 1)
        res[tag]["prepared_bytes"] = pkg.prepared_bytes(K, N, G)
        del preps
        torch.cuda.empty_cache()

    layout_case("prepared_c0_gptq_sym_m1_k4096_n4096", "gptq_sym", 1, 4096, 4096, 128, 60, 1000)
    for M in (1, 4, 8):
        layout_case(f"prepared_c1_awq_m{M}_k4096_n14336", "awq", M, 4096, 14336, 128, 20, 1000)
        layout_case(f"prepared_c1_awq_m{M}_k14336_n4096", "awq", M, 14336, 4096, 128, 20, 1000)
    layout_case("prepared_c3_awq_m2048_k4096_n14336", "awq", 2048, 4096, 14336, 128, 2, 300)
    layout_case("prepared_c3_awq_m2048_k14336_n4096", "awq", 2048, 14336, 4096, 128, 2, 300)

    # one GPU's share of an 8-way tensor-parallel MLP at its real shape: gate/up split by
    # columns (N / 8 = 1792), down split by rows (K / 8 = 1792); 150 weight sets (> 512 MB)
    for M in (1, 8):
        gemm_case(f"tp8_c1_awq_m{M}_k4096_n1792", "awq", M, 4096, 1792, 128, 150, 1000)
        gemm_case(f"tp8_c1_awq_m{M}_k1792_n4096", "awq", M, 1792, 4096, 128, 150, 1000)
    gemm_case("tp8_c3_awq_m2048_k4096_n1792", "awq", 2048, 4096, 1792, 128, 2, 300)
    gemm_case("tp8_c3_awq_m2048_k1792_n4096", "awq", 2048, 1792, 4096, 128, 2, 300)

    # the reference-named typed entry point (its 19-parameter list, dense strides) at C1 / C3,
    # called through the C ABI and launched by name through the DeviceRuntime backend
    # (hiprt_launch of awq_gemm_int4_typed from w4a16_typed.hsaco, grid (cdiv(M,64),
    # cdiv(N,64), 1) x 256 threads, the 19 arguments + 2 scratch pointers)
    rt = pkg.HipRuntime(0)
    hs_mod = rt.load_module(pkg.typed_module_bytes())
    scratch = torch.empty(1, dtype=torch.uint8, device=dev)

    def typed_case(tag, M, K, N, n_sets, calls, hiprt=False):
        G = 128
        sets = make_weight_sets(torch, "awq", K, N, G, n_sets, dev, seed=zlib.crc32(tag.encode()))
        x = torch.randn((M, K), device=dev, generator=gen).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        st = [K, 1, N // 8, 1, N, 1, N // 8, 1, N, 1]
        A = pkg.KernelArg
        args = [[A.ptr(x), A.ptr(qw), A.ptr(sc), A.ptr(qz), A.ptr(out)] +
                [A.i32(v) for v in (M, N, K, G, *st)] + [A.ptr(scratch), A.ptr(scratch)]
                for qw, sc, qz in sets]
        grid = (-(-M // 64), -(-N // 64), 1)

        def fn(i):
            if hiprt:
                rt.launch(hs_mod, "awq_gemm_int4_typed", grid, (256, 1, 1), 0, None, args[i % n_sets])
            else:
                qw, sc, qz = sets[i % n_sets]
                pkg.awq_gemm_int4_typed(x, qw, sc, qz, out, M, N, K, G, *st)
        ms = time_calls(torch, fn, GRAPH_CALLS, 10, stream, n_sets, batch_calls=calls)[1]
        record(tag, "awq", M, K, N, G, ms,
               ("hiprt->" if hiprt else "typed->") + pkg.typed_plan("awq", M, N, K, G, st))
        del sets, args

    typed_case("typed_awq_gemm_int4_m1_k4096_n14336", 1, 4096, 14336, 20, 1000)
    typed_case("typed_awq_gemm_int4_m2048_k4096_n14336", 2048, 4096, 14336, 2, 300)
    typed_case("hiprt_awq_gemm_int4_typed_m1_k4096_n14336", 1, 4096, 14336, 20, 1000, hiprt=True)
    typed_case("hiprt_awq_gemm_int4_typed_m2048_k4096_n14336", 2048, 4096, 14336, 2, 300, hiprt=True)
    rt.unload_module(hs_mod)
    rt.close()

    # config 4: fused MoE layer, T=512, 8 experts, top-2, K=4096, I=14336, GPTQ G=128
    L = moe_layer(torch, dev, gen)
    T, E, topk, K, I = L["T"], L["E"], L["topk"], L["K"], L["I"]
    w13, w2, x, logits = L["w13"], L["w2"], L["x"], L["logits"]
    out = torch.empty((T, K), dtype=torch.float16, device=dev)
    flops = 2.0 * T * topk * (K * 2 * I + I * K)
    for bm in (64, 128):
        ws = torch.empty(pkg.lib().w4a16_fused_moe_workspace_size(T, E, topk, I, K, bm),
                         dtype=torch.uint8, device=dev)
        ms = time_calls(torch, lambda i: pkg.fused_moe(x, logits, w13, w2, topk=topk, block_m=bm,
                                                       out=out, workspace=ws),
                        10, 5, stream, 1, batch_calls=20, graph_calls=10, n_graphs=1)[1]
        res[f"c4_fused_moe_block_m{bm}"] = {
            "ms_per_layer": round(ms, 3), "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_mfma": round(flops / (ms * 1e-3) / 1e12 / FP16_DENSE_PEAK_TFLOPS, 4)}
        progress(f"fused moe block_m={bm}: {ms:.3f} ms")
        del ws
    # the same layer on the experts in the prepared layout (w4a16_prepare_layout per expert,
    # once; timed: w4a16_fused_moe_prepared only)
    w13p = pkg.prepare_layout_experts(*w13, fmt="gptq", group_size=L["G"], zero_offset=1)
    w2p = pkg.prepare_layout_experts(*w2, fmt="gptq", group_size=L["G"], zero_offset=1)
    ws = torch.empty(pkg.lib().w4a16_fused_moe_workspace_size(T, E, topk, I, K, 64),
                     dtype=torch.uint8, device=dev)
    ms = time_calls(torch, lambda i: pkg.fused_moe_prepared(x, logits, w13p, w2p, topk=topk, block_m=64,
                                                            out=out, workspace=ws),
                    10, 5, stream, 1, batch_calls=20, graph_calls=10, n_graphs=1)[1]
    res["c4_fused_moe_prepared"] = {
        "ms_per_layer": round(ms, 3), "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
        "frac_mfma": round(flops / (ms * 1e-3) / 1e12 / FP16_DENSE_PEAK_TFLOPS, 4)}
    progress(f"fused moe on prepared experts: {ms:.3f} ms")
    del ws, w13p, w2p
    del w13, w2, L
    torch.cuda.empty_cache()
    res["achievable"] = achievable_refs(torch, dev, stream)
    res["achievable"].update(dequant_then_mm_refs(torch, pkg, dev, stream, gen))
    return res


def achievable_refs(torch, dev, stream):
    """Measured HBM references on this GPU, beside the spec peak: a device-to-device copy
    (bytes read + written), a read-only fp32 sum of 512 MiB, and the per-launch floor of a
    one-element kernel replayed from HIP graphs like the GEMM calls. (The MFMA references, torch's
    fp16 GEMM at config 3's shapes, come from dequant_then_mm_refs, timed like the GEMMs.)"""
    out = {}
    n = 512 << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()

    def t_ms(fn, reps):
        with torch.cuda.stream(stream):
            fn(); fn()
        torch.cuda.synchronize()
        st, sp = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            fn()
            st.record(stream)
            for _ in range(reps):
                fn()
            sp.record(stream)
        torch.cuda.synchronize()
        return st.elapsed_time(sp) / reps

    ms = t_ms(lambda: b.copy_(a), 20)
    out["d2d_copy_GBps"] = round(2 * n / (ms * 1e-3) / 1e9, 1)
    af = a.view(torch.float32)      # bytes of 1: small normal floats
    ms = t_ms(lambda: torch.sum(af), 20)
    out["read_sum_f32_GBps"] = round(n / (ms * 1e-3) / 1e9, 1)
    del a, b, af
    # per-launch floor of a kernel in a graph replay, timed like the GEMMs: one-element add
    tiny = torch.zeros(1, dtype=torch.int32, device=dev)
    out["graph_launch_floor_us"] = round(
        time_calls(torch, lambda i: tiny.add_(1), 1000, 10, stream, 1)[1] * 1e3, 2)
    progress(f"achievable references: {out}")
    return out


def n_sweep(args) -> int:
    """The headline kernel (prepared layout, M = 1, K = 4096, AWQ) at several N, timed as the
    headline is (graph replays, median of 5 batches of 1000 calls, weight sets rotated over at
    least 700 MB), then t = a + b N by least squares: a is the fixed cost of a call, b the
    marginal cost per column, and bytes per column / b the marginal streaming rate."""
    import numpy as np
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    fmt, M, K, _, G = HEADLINE
    ns_, ts_ = [], []
    for N in (int(v) for v in args.n_sweep.split(",")):
        per_set = algorithmic_bytes(fmt, M, K, N, G)
        n_sets = max(8, int(700e6 // per_set) + 1)
        sets = make_weight_sets(torch, fmt, K, N, G, n_sets, dev, seed=zlib.crc32(b"sweep%d" % N))
        preps = [pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G) for qw, sc, qz in sets]
        del sets
        x = torch.randn((M, K), device=dev).half()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        ms = time_calls(torch, lambda i: pkg.gemm_prepared(x, preps[i % n_sets], out=out), 2000, 50,
                        stream, n_sets)[1]
        ns_.append(N)
        ts_.append(ms * 1e3)
        print(f"N={N} strips={N // 16} per_cu={N / 16 / 256:.2f} us={ms * 1e3:.3f} "
              f"GBps={per_set / (ms * 1e-3) / 1e9:.0f}", flush=True)
        del preps
        torch.cuda.empty_cache()
    if len(ns_) >= 2:
        n_arr, t_arr = np.array(ns_, dtype=float), np.array(ts_)
        b, a = np.polyfit(n_arr, t_arr, 1)
        per_col = algorithmic_bytes(fmt, M, K, 1000, G) / 1000.0   # x and out are per call
        print(f"fit: t = {a:.3f} us + {b * 1e3:.4f} us per 1000 columns; marginal "
              f"{per_col / (b * 1e-6) / 1e12:.2f} TB/s; residuals "
              f"{np.round(t_arr - (a + b * n_arr), 3).tolist()}", flush=True)
    tiny = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"graph-replay floor of a one-element kernel: "
          f"{time_calls(torch, lambda i: tiny.add_(1), 1000, 10, stream, 1)[1] * 1e3:.2f} us", flush=True)
    return 0


def dequant_then_mm_refs(torch, pkg, dev, stream, gen):
    """The unfused dense path at config 3's shapes: this library's dequantisation of the AWQ
    weights to fp16 [K, N], then torch's fp16 GEMM (hipBLASLt / rocBLAS), per call, against
    which the fused prefill kernel is compared (rotated weight sets, graph replays, as for the
    GEMMs); and torch's fp16 GEMM alone timed the same way."""
    out = {}
    for K, N in ((4096, 14336), (14336, 4096)):
        M = 2048
        sets = make_weight_sets(torch, "awq", K, N, 128, 4, dev, seed=zlib.crc32(b"deq%d" % K))
        x = torch.randn((M, K), device=dev, generator=gen).half()
        w16 = torch.empty((K, N), dtype=torch.float16, device=dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        lib = pkg.lib()

        def fn(i):
            qw, sc, qz = sets[i % len(sets)]
            pkg.check(lib.w4a16_dequant(pkg._stream(qw), pkg.FMT_AWQ, pkg._ptr(qw), pkg._ptr(sc),
                                        pkg._ptr(qz), None, pkg._ptr(w16), K, N, 128, 1, 0))
            torch.mm(x, w16, out=y)
        ms = time_calls(torch, fn, 20, 5, stream, len(sets), batch_calls=40, graph_calls=10,
                        n_graphs=2)[1]
        out[f"dequant_then_torch_mm_m{M}_k{K}_n{N}_us"] = round(ms * 1e3, 1)
        # the fp16 GEMM alone, timed the same way (graph replays), over 4 rotated fp16 weights
        ws16 = [torch.randn((K, N), device=dev, generator=gen).half() for _ in range(4)]
        ms = time_calls(torch, lambda i: torch.mm(x, ws16[i % 4], out=y), 20, 5, stream, 4,
                        batch_calls=40, graph_calls=10, n_graphs=2)[1]
        out[f"torch_fp16_mm_m{M}_k{K}_n{N}_us"] = round(ms * 1e3, 1)
        out[f"torch_fp16_mm_m{M}_k{K}_n{N}_TFLOPs"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)
        del sets, x, w16, y, ws16
    torch.cuda.empty_cache()
    progress(f"dequant then fp16 GEMM: {out}")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--sets", type=int, default=20, help="distinct weight buffers rotated")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-traffic", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--headline-only", action="store_true",
                    help="time the headline and exit (no JSON line): for kernel-trace profiles "
                         "whose statistics should cover the cold headline dispatches only")
    ap.add_argument("--n-sweep", default="",
                    help="comma-separated N values: time the headline kernel (prepared layout, "
                         "M=1, K=4096) at each N, fit fixed + per-column cost, and exit (no JSON "
                         "line): the fixed and marginal cost of the headline call")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-workload", default="headline", choices=sorted(PMC_WORKLOADS),
                    help="workload of a --pmc-child or --pmc-report run (for counter profiles)")
    ap.add_argument("--pmc-report", action="store_true",
                    help="run counter passes over --pmc-workload and print their per-kernel "
                         "means as one JSON line (FETCH_SIZE/WRITE_SIZE traffic by default)")
    ap.add_argument("--pmc-counters", default="",
                    help="counter passes for --pmc-report: groups separated by ';', counters "
                         "within a group by spaces (one rocprofv3 run per group)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; the kernels "
              "run on one GPU's share of a sharded layer", file=sys.stderr)
        return 2
    if args.pmc_child:
        return pmc_child(args)
    if args.pmc_report:
        return pmc_report(args)

    if args.n_sweep:
        return n_sweep(args)

    # counter passes run first, in child processes, before this process touches the GPU
    traffic, traffic_detail = (None, {"traffic_note": "skipped (--no-traffic)"})
    if not args.no_traffic:
        try:
            traffic, traffic_detail = measure_traffic(args)
            progress(f"counter passes done: traffic={traffic}")
        except (RuntimeError, OSError, KeyError, ValueError) as e:
            traffic, traffic_detail = None, {"traffic_note": f"counter pass unusable: {e}"}

    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    fmt, M, K, N, G = HEADLINE
    sets = make_weight_sets(torch, fmt, K, N, G, args.sets, dev, seed=0x5EED0001)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x5EED0001)
    x = torch.randn((M, K), device=dev, generator=gen).half()
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    stream = torch.cuda.Stream(device=dev)
    n_sets = len(sets)
    nbytes = algorithmic_bytes(fmt, M, K, N, G)

    # The AWQ checkpoint of every weight set is rewritten once into the prepared layout
    # (w4a16_prepare_layout, the load-time step); one such call is timed on its own.
    qw, sc, qz = sets[0]
    pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    pkg.prepare_layout(qw, sc, qz, fmt=fmt, group_size=G)
    ev1.record()
    torch.cuda.synchronize()
    prepare_us = ev0.elapsed_time(ev1) * 1e3
    preps = [pkg.prepare_layout(q, s_, z, fmt=fmt, group_size=G) for q, s_, z in sets]
    torch.cuda.synchronize()

    def headline_call(i):
        pkg.gemm_prepared(x, preps[i % n_sets], out=out)

    def checkpoint_call(i):
        q, s_, z = sets[i % n_sets]
        pkg.gemm(x, q, s_, z, fmt=fmt, group_size=G, out=out)

    # timed region: exactly args.steps calls; then 5 further batches of 1000 for the median
    ms, ms_med, batch_ms, wall = time_calls(torch, headline_call, args.steps, args.warmup, stream,
                                            n_sets, batches=5, batch_calls=1000, exact_direct=True)
    if args.headline_only:
        progress(f"headline only: {ms * 1e3:.3f} us/call exact, {ms_med * 1e3:.3f} median")
        return 0
    ms_direct = time_direct(torch, headline_call, min(args.steps, 1000), stream)
    # warm single buffer (Infinity-Cache resident), reported separately
    ms_warm = time_calls(torch, lambda i: pkg.gemm_prepared(x, preps[0], out=out), 1000, 50,
                         stream, 1)[1]
    # the same workload on the checkpoint layout as stored (w4a16_gemm, split-K GEMV)
    ms_ckpt = time_calls(torch, checkpoint_call, 1000, 50, stream, n_sets)[1]
    kernel_ckpt = pkg.plan(fmt, M, N, K, G)
    gbs = nbytes / (ms * 1e-3) / 1e9
    progress(f"headline: {ms * 1e3:.2f} us/call over exactly {args.steps} calls, {gbs:.1f} GB/s; "
             f"median of 5 x 1000 calls {ms_med * 1e3:.2f} us; checkpoint layout "
             f"{ms_ckpt * 1e3:.2f} us")

    result = {
        "metric": "W4A16 GEMM GB/s (M=1) and TFLOP/s (M=2048), % of MI355X roofline",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded torch RNG on device: uniform int4 nibbles, scales U[0.002,0.02], x~N(0,1))",
        "config": {"workload": f"AWQ int4 GEMV M={M} K={K} N={N} group_size={G} (config 1, M=1): "
                               f"AWQ checkpoint weights prepared once (w4a16_prepare_layout), then "
                               f"w4a16_gemm_prepared per step",
                   "kernel": "prepared/gemv (gemv_prep_mfma_kernel)", "weight_sets_rotated": n_sets,
                   "rotated_footprint_MB": round(n_sets * pkg.prepared_bytes(K, N, G) / 1e6, 1),
                   "prepare_once_us": round(prepare_us, 1),
                   "timing": (f"HIP events on the launch stream around exactly {args.steps} calls "
                              + (f"launched directly, enqueued behind {GRAPH_CALLS * 10} untimed calls "
                                 f"replayed from HIP graphs" if args.steps <= DIRECT_MAX_STEPS else
                                 f"replayed from HIP graphs, untimed replays enqueued ahead of the "
                                 f"start event"))},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": nbytes, **traffic_detail},
        "extra": {"median_of_5_batches_us": round(ms_med * 1e3, 3),
                  "median_of_5_batches_GBps": round(nbytes / (ms_med * 1e-3) / 1e9, 1),
                  "batch_us": [round(b * 1e3, 3) for b in batch_ms],
                  "batch_calls": 1000,
                  "direct_launch_us_per_call": round(ms_direct * 1e3, 2),
                  "direct_launch_GBps": round(nbytes / (ms_direct * 1e-3) / 1e9, 1),
                  "warm_single_buffer_us": round(ms_warm * 1e3, 2),
                  "warm_single_buffer_GBps": round(nbytes / (ms_warm * 1e-3) / 1e9, 1),
                  "timed_wall_s": round(wall, 4),
                  "checkpoint_layout": {"kernel": kernel_ckpt, "us_per_call": round(ms_ckpt * 1e3, 2),
                                        "GBps": round(nbytes / (ms_ckpt * 1e-3) / 1e9, 1),
                                        "frac_hbm": round(nbytes / (ms_ckpt * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                        "entry": "w4a16_gemm on the AWQ checkpoint as stored"}},
    }
    if not args.no_extra:
        del sets, preps
        torch.cuda.empty_cache()
        result["extra"].update(extras(torch, pkg, dev, stream, args))

    if not args.no_cpu_baseline:
        qw, sc, qz = (t.cpu().numpy() for t in make_weight_sets(torch, fmt, K, N, G, 1, dev,
                                                                 seed=0x5EED0001)[0])
        xh = x.cpu().numpy()
        med, n, med_dq, n_dq, threads = cpu_baseline(2, xh, qw, sc, qz, M, K, N, G, args.cpu_budget)
        result["cpu_baseline"] = {
            "value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} whole calls of the same M=1 K={K} N={N} AWQ workload (median "
                      f"{med * 1e3:.1f} ms/call: dequant + fp32 matmul, OpenMP); host "
                      f"{cpu_model()}, nproc={os.cpu_count()}",
            "dequant_only_ms": round(med_dq * 1e3, 2),
            "dequant_only_GBps": round(nbytes / med_dq / 1e9, 3),
            "dequant_only_sample": f"{n_dq} dequantisations of the same weights to fp16 [K, N]"}

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
