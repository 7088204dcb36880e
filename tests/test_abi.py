"""CPU-side checks of the C ABI: the library loads, exports every symbol include/w4a16.h
declares, and rejects bad arguments before touching the GPU (no compute calls here)."""
import ctypes
import json
import os
import re
import subprocess

import pytest

from helpers import ROOT, pkg

HEADER = os.path.join(ROOT, "include", "w4a16.h")


def declared_functions():
    text = open(HEADER).read()
    return re.findall(r"W4A16_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    P = pkg()
    L = P.lib()
    names = declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/w4a16.h but not exported"
    assert set(names) == set(P.EXPORTED)
    out = subprocess.run(["nm", "-D", "--defined-only", P.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(names) <= exported


def _c_param_counts():
    """Parameter count of every W4A16_API function in include/w4a16.h."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"W4A16_API\s+[\w\s\*]+?\b(\w+)\s*\(([^)]*)\)", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _rust_extern_fns(text):
    """(name, parameter count) of every fn in the `extern "C" { ... }` blocks of Rust text."""
    fns = []
    for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"\bfn\s+(\w+)\s*\(([^)]*)\)", block, flags=re.S):
            args = m.group(2).strip().rstrip(",")
            fns.append((m.group(1), 0 if not args else args.count(",") + 1))
    return fns


@pytest.mark.parametrize("source", ["rust/triton-runtime-hip/src/lib.rs", "INTEGRATION.md"])
def test_rust_ffi_block_matches_the_header(source):
    """The Rust backend cannot be compiled in this image (no cargo): its FFI declarations are
    checked here instead. Every libw4a16 function they bind is declared in include/w4a16.h
    with the same number of parameters (the hiprt_* runtime calls included)."""
    c = _c_param_counts()
    fns = _rust_extern_fns(open(os.path.join(ROOT, source)).read())
    assert len(fns) >= 15, source
    for name, n in fns:
        assert name in c, f"{source}: fn {name} is not declared in include/w4a16.h"
        assert c[name] == n, f"{source}: fn {name} takes {n} parameters, the header {c[name]}"


def test_version_and_empty_error():
    P = pkg()
    assert "gfx950" in P.version()


def _gemm(P, **over):
    a = dict(stream=None, fmt=P.FMT_AWQ, x=1, qw=1, sc=1, qz=1, g=None, out=1, M=1, N=4096,
             K=4096, G=128, zo=1)
    a.update(over)
    p = lambda v: None if v is None else ctypes.c_void_p(v)
    return P.lib().w4a16_gemm(a["stream"], a["fmt"], p(a["x"]), p(a["qw"]), p(a["sc"]), p(a["qz"]),
                              p(a["g"]), p(a["out"]), a["M"], a["N"], a["K"], a["G"], a["zo"])


@pytest.mark.parametrize("over,needle", [
    (dict(x=None), "null pointer"),
    (dict(qz=None), "qzeros is required"),
    (dict(K=4000), "multiple of group_size"),
    (dict(N=4100), "multiple of 8"),
    (dict(M=0), "sizes must be positive"),
    (dict(G=0), "sizes must be positive"),
    (dict(fmt=7), "unknown weight format"),
    (dict(fmt=0, K=4100, G=4100), "multiple of 8 for GPTQ"),
    (dict(fmt=0, zo=-1), "gptq_zero_offset"),
    (dict(fmt=0, zo=17), "gptq_zero_offset"),
])
def test_gemm_argument_errors_before_any_hip_call(over, needle):
    P = pkg()
    rc = _gemm(P, **over)
    assert rc == P.ERR_INVALID_ARG
    assert needle in P.lib().w4a16_last_error().decode()


def test_gptq_sym_does_not_need_qzeros():
    P = pkg()
    k = ctypes.c_int()
    assert P.lib().w4a16_gemm_plan(P.FMT_GPTQ_SYM, 1, 4096, 4096, 128, 0, ctypes.byref(k)) == 0


def test_plan_regimes():
    P = pkg()
    assert P.plan("awq", 1, 14336, 4096, 128) == "gemv"
    assert P.plan("awq", 1, 4096, 14336, 128) == "gemv"
    assert P.plan("gptq_sym", 1, 4096, 4096, 128) == "gemv"
    assert P.plan("gptq", 1, 4096, 4096, 128, has_g_idx=True) != "gemv"


def test_dequant_reference_arg_check():
    P = pkg()
    rc = P.lib().dequant_int4_to_fp16(None, ctypes.c_void_p(1), ctypes.c_void_p(1),
                                      ctypes.c_void_p(1), ctypes.c_void_p(16), 4096, 4096, 128, 511)
    assert rc == P.ERR_INVALID_ARG and "n_div_8" in P.lib().w4a16_last_error().decode()


def test_runtime_null_and_launch_config_errors():
    P = pkg()
    L = P.lib()
    assert L.hiprt_create(0, None) == P.ERR_INVALID_ARG
    assert L.hiprt_module_load(None, None, 0, None) == P.ERR_INVALID_ARG
    g = (ctypes.c_uint32 * 3)(1, 1, 1)
    b = (ctypes.c_uint32 * 3)(2048, 1, 1)
    # a fake non-null ctx/module is never dereferenced: the launch config is checked first
    rc = L.hiprt_launch(ctypes.c_void_p(8), ctypes.c_void_p(8), b"k", g, b, 0, None, None, 0)
    assert rc == P.ERR_LAUNCH_CONFIG
    z = (ctypes.c_uint32 * 3)(0, 1, 1)
    assert L.hiprt_launch(ctypes.c_void_p(8), ctypes.c_void_p(8), b"k", z, g, 0, None, None, 0) \
        == P.ERR_LAUNCH_CONFIG
    big = (ctypes.c_uint32 * 3)(64, 1, 1)
    assert L.hiprt_launch(ctypes.c_void_p(8), ctypes.c_void_p(8), b"k", g, big, 200 * 1024, None,
                          None, 0) == P.ERR_LAUNCH_CONFIG


def test_runtime_backend_disabled_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    P = pkg()
    with pytest.raises(P.BackendDisabled):
        P.HipRuntime(0)


def test_typed_code_object_names_and_metadata():
    P = pkg()
    data = P.typed_module_bytes()
    assert data[:4] == b"\x7fELF"
    out = subprocess.run(["readelf", "-sW", P.HSACO_PATH], capture_output=True, text=True,
                         check=True).stdout
    for name in ("w4a16_gptq_gemm_typed", "awq_gemm_int4_typed"):
        assert re.search(rf"\b{name}\b", out), name
    meta = P.typed_module_meta()
    names = {k["name"] for k in meta["kernels"]}
    assert names == {"w4a16_gptq_gemm_typed", "awq_gemm_int4_typed"}
    for k in meta["kernels"]:
        assert k["num_warps"] * 32 == k["threads_per_block"] == 256
        assert k["params"] == 21


def _disassemble_tu(obj, tmp_path):
    """gfx950 disassembly of one of our own build's translation units."""
    fb, dev = tmp_path / "fb.bin", tmp_path / "dev.o"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, str(fb)],
                   check=True)
    subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={fb}",
                    f"--output={dev}"], check=True)
    dis = subprocess.run(["/opt/rocm/llvm/bin/llvm-objdump", "-d", str(dev)],
                         capture_output=True, text=True, check=True).stdout
    funcs = {}
    for chunk in re.split(r"\n(?=[0-9a-f]+ <)", dis):
        m = re.match(r"[0-9a-f]+ <([^>]+)>", chunk)
        if m:
            funcs[m.group(1)] = chunk
    return funcs


def test_kernel_choice_evidence_in_isa(tmp_path):
    """The VALU decode GEMVs use v_dot2 and no MFMA; the AWQ matrix-core GEMVs (block-diagonal
    and row-paired) and the strided GEMM use fp16 MFMA, the strided GEMM's bfloat16 instances
    bf16 MFMA. Every VALU GEMV comes in two hand-off variants (device scope, XCD-local)."""
    bdir = os.path.join(ROOT, "triton-rs_amd", "_build")
    gemv_o, strided_o = os.path.join(bdir, "kernels_gemv.o"), os.path.join(bdir, "kernels_strided.o")
    if not (os.path.exists(gemv_o) and os.path.exists(strided_o)):
        pytest.skip("build objects not present (run build first)")
    kernels = _disassemble_tu(gemv_o, tmp_path)
    gemv = {k: v for k, v in kernels.items() if "gemv_" in k and "mfma" not in k
            and "rows" not in k and "probe" not in k}
    gemv_mc = {k: v for k, v in kernels.items() if "gemv_awq_mfma_kernel" in k
               or "gemv_awq_rows_kernel" in k}
    strided = {k: v for k, v in _disassemble_tu(strided_o, tmp_path).items()
               if "strided_gemm_kernel" in k}
    assert len(gemv) >= 24 and len(gemv_mc) >= 8 and len(strided) == 7   # 6 + prepared (fp16)
    for name, body in gemv.items():
        assert "v_mfma" not in body, name
        assert "v_dot2" in body, name
    for name, body in gemv_mc.items():   # the row-paired kernel also comes in bf16
        bf16 = "DF16b" in name
        assert ("v_mfma_f32_16x16x32_bf16" if bf16 else "v_mfma_f32_16x16x32_f16") in body, name
    for name, body in strided.items():
        bf16 = "DF16b" in name        # the __bf16 element type in the mangled name
        assert ("v_mfma_f32_16x16x32_bf16" if bf16 else "v_mfma_f32_16x16x32_f16") in body, name
        assert ("v_cvt_pk_bf16_f32" in body) == bf16, name


def test_prepared_kernels_isa(tmp_path):
    """Prepared-layout kernels: the M = 1 and M = 2..8 GEMVs and the small-batch kernel run
    their dot products on fp16 MFMA (shifts and v_and_or_b32 per word feed them), the
    group-size-32/64 GEMV on v_dot2 without MFMA; no split-K atomics anywhere in them, and no
    scratch (spilled registers) in the small-batch kernels."""
    o = os.path.join(ROOT, "triton-rs_amd", "_build", "prepared.o")
    if not os.path.exists(o):
        pytest.skip("build objects not present (run build first)")
    k = _disassemble_tu(o, tmp_path)
    mf = {n: b for n, b in k.items() if "gemv_prep_mfma_kernel" in n or "gemv_prep_rows_kernel" in n}
    va = {n: b for n, b in k.items() if "gemv_prep_valu_kernel" in n}
    assert len(mf) >= 6 and len(va) >= 3
    for n, b in mf.items():
        assert "v_mfma_f32_16x16x32_f16" in b and "v_and_or_b32" in b, n
        assert "atomic" not in b, n
    for n, b in va.items():
        assert "v_mfma" not in b and "v_dot2" in b and "atomic" not in b, n
    fr = {n: b for n, b in k.items() if "gemm_prep_frag_kernel" in n}
    assert len(fr) >= 20
    for n, b in fr.items():   # the nibble pairs by v_and_or_b32, or v_or3_b32 after a mask
        assert "v_mfma_f32_16x16x32_f16" in b and ("v_and_or_b32" in b or "v_or3_b32" in b), n
        assert "atomic" not in b and "scratch_" not in b and "buffer_store" not in b, n


def test_bf16_flag_plans_and_is_refused_elsewhere():
    """W4A16_BF16 plans the VALU GEMV up to 4 rows, the small-batch kernel up to 64 and the
    pipelined prefill beyond (act-order: the small-batch kernel, then the group-order prefill
    route), the generic kernel for other shapes; entry points without a bfloat16 instantiation report the
    flagged value as an unknown format (no GPU call)."""
    P = pkg()
    L = P.lib()
    k = ctypes.c_int(0)

    def plan(fmt, M, N, K, gidx=0):
        assert L.w4a16_gemm_plan(fmt, M, N, K, 128, gidx, ctypes.byref(k)) == P.OK
        return P.KERNELS[k.value]
    for M, N, K, want in ((1, 14336, 4096, "gemv"), (4, 4096, 14336, "gemv"),
                          (16, 6144, 4096, "skinny"), (64, 6144, 4096, "skinny"),
                          (65, 6144, 4096, "prefill"), (2048, 4096, 14336, "prefill"),
                          (33, 136, 384, "strided")):
        assert plan(P.FMT_AWQ | P.BF16, M, N, K) == want, (M, N, K)
        assert plan(P.FMT_GPTQ | P.BF16, M, N, K) == want, (M, N, K)
    # 5..8 rows: the row-paired AWQ GEMV, GPTQ the small-batch kernel
    assert plan(P.FMT_AWQ | P.BF16, 8, 4096, 14336) == "gemv"
    assert plan(P.FMT_GPTQ | P.BF16, 8, 4096, 14336) == "skinny"
    assert plan(P.FMT_GPTQ | P.BF16, 16, 6144, 4096, gidx=1) == "skinny"
    assert plan(P.FMT_GPTQ | P.BF16, 2048, 6144, 4096, gidx=1) == "prefill"
    assert plan(P.FMT_GPTQ | P.BF16, 33, 136, 384, gidx=1) == "strided"
    assert plan(P.FMT_AWQ, 1, 14336, 4096) == "gemv"
    assert L.w4a16_gemm_plan(P.FMT_AWQ | 0x200, 1, 512, 512, 128, 0, ctypes.byref(k)) == \
        P.ERR_INVALID_ARG
    assert L.w4a16_prepare_act_order(None, P.FMT_GPTQ | P.BF16, None, None, 1024, 256, 128,
                                     None, None) == P.ERR_INVALID_ARG
    assert "fmt" in L.w4a16_last_error().decode()


def test_bf16_fast_kernels_isa(tmp_path):
    """The bfloat16 instances of the small-batch and prefill kernels run bf16 MFMA on weights
    rounded with v_cvt_pk_bf16_f32 (from v_cvt_f32_ubyte nibble conversions), the bf16 VALU
    GEMVs v_dot2c_f32_bf16 without MFMA, and none spills; their fp16 twins have none of it."""
    bdir = os.path.join(ROOT, "triton-rs_amd", "_build")
    gv = os.path.join(bdir, "kernels_gemv.o")
    objs = [os.path.join(bdir, f) for f in ("kernels_skinny.o", "kernels_prefill.o")]
    if not all(os.path.exists(o) for o in objs + [gv]):
        pytest.skip("build objects not present (run build first)")
    gk = {n: b for n, b in _disassemble_tu(gv, tmp_path).items()
          if "gemv_awq_kernel" in n or "gemv_gptq_kernel" in n}
    gbf = {n: b for n, b in gk.items() if "DF16b" in n}
    assert len(gbf) >= 60, len(gbf)
    for n, b in gk.items():
        bf = "DF16b" in n
        assert ("v_dot2c_f32_bf16" in b) == bf and ("v_dot2c_f32_f16" in b) != bf, n
        assert "v_mfma" not in b and "scratch_" not in b, n
    if not all(os.path.exists(o) for o in objs):
        pytest.skip("build objects not present (run build first)")
    seen = 0
    for o, name in zip(objs, ("skinny_kernel", "prefill_dma_kernel")):
        ks = {n: b for n, b in _disassemble_tu(o, tmp_path).items() if name in n}
        bf = {n: b for n, b in ks.items() if "DF16b" in n}
        assert len(bf) >= (48 if name == "skinny_kernel" else 18), (name, len(bf))
        for n, b in bf.items():
            assert "v_mfma_f32_16x16x32_bf16" in b and "v_mfma_f32_16x16x32_f16" not in b, n
            assert "v_cvt_pk_bf16_f32" in b and "v_cvt_f32_ubyte" in b, n
            assert "scratch_" not in b, n
            seen += 1
        for n, b in ks.items():
            if "DF16b" not in n:
                assert "v_mfma_f32_16x16x32_bf16" not in b and "v_cvt_pk_bf16_f32" not in b, n
    assert seen >= 66


def test_moe_argument_errors():
    P = pkg()
    L = P.lib()
    v = ctypes.c_void_p(256)
    assert L.w4a16_moe_route(None, None, 4, 8, 2, 1, v, v) == P.ERR_INVALID_ARG
    assert L.w4a16_moe_route(None, v, 4, 8, 9, 1, v, v) == P.ERR_INVALID_ARG      # topk > E
    assert L.w4a16_moe_route(None, v, 4, 300, 2, 1, v, v) == P.ERR_UNSUPPORTED   # E > 256
    # capacity below pairs + E * (block_m - 1)
    assert L.w4a16_moe_align(None, v, 1024, 8, 64, 1024, v, v, v) == P.ERR_INVALID_ARG
    assert "capacity" in L.w4a16_last_error().decode()
    # grouped GEMM shape limits
    rc = L.w4a16_moe_gemm(None, 0, v, 2, v, v, v, 0, 0, 0, 8, v, v, v, v, 1024, 1004, 4096, 128,
                          64, 1536, 1)
    assert rc == P.ERR_INVALID_ARG        # N % 8
    rc = L.w4a16_moe_gemm(None, 0, v, 2, v, v, v, 0, 0, 0, 8, v, v, v, v, 1024, 1032, 4096, 128,
                          64, 1536, 1)
    assert rc == P.ERR_UNSUPPORTED        # N % 256
    rc = L.w4a16_moe_gemm(None, 0, v, 2, v, v, v, 0, 0, 0, 0, v, v, v, v, 1024, 1024, 4096, 128,
                          64, 1536, 1)
    assert rc == P.ERR_INVALID_ARG        # num_experts < 1
    assert L.fused_silu_mul_interleaved_f16(None, v, v, 0, 250) == P.ERR_INVALID_ARG
    assert L.fused_silu_mul_interleaved_f16(None, v, v, 100, -1) == P.ERR_INVALID_ARG
    # any inter and a total that is not a multiple of it are the reference's domain
    assert L.fused_silu_mul_interleaved_f16(None, v, v, 100, 0) == P.OK
    assert L.fused_silu_mul_interleaved_f32(None, v, v, 0, 250) == P.ERR_INVALID_ARG
    assert L.fused_silu_mul_interleaved_f32(None, v, v, 100, -1) == P.ERR_INVALID_ARG
    assert L.fused_silu_mul_interleaved_f32(None, None, v, 100, 10) == P.ERR_INVALID_ARG
    assert L.fused_silu_mul_interleaved_f32(None, v, v, 100, 0) == P.OK
    assert L.w4a16_fused_moe_workspace_size(512, 8, 2, 14336, 4096, 64) > 512 * 2 * 14336 * 2
    ws = L.w4a16_fused_moe_workspace_size(512, 8, 2, 14336, 4096, 64)
    rc = L.w4a16_fused_moe(None, 0, v, v, 512, 4096, 14336, 8, 2, 1, v, v, v, v, v, v, 128, 64, 1,
                           v, ws - 1, v)
    assert rc == P.ERR_INVALID_ARG and "workspace" in L.w4a16_last_error().decode()


def _dense_strides(fmt, m, n, k):
    return [k, 1, n // 8 if fmt == "awq" else n, 1, n, 1, n // 8, 1, n, 1]


@pytest.mark.parametrize("fmt,m,n,k,expect", [
    ("awq", 1, 14336, 4096, "gemv"), ("awq", 4, 4096, 14336, "gemv"),
    ("gptq", 16, 6144, 4096, "skinny"), ("awq", 2048, 14336, 4096, "prefill"),
    ("gptq", 1, 4096, 4096, "gemv"),
])
def test_typed_entry_points_route_dense_layouts_to_the_planner(fmt, m, n, k, expect):
    """The reference-named typed entry points take w4a16_gemm's kernels for dense row-major
    operands, and the generic strided kernel otherwise."""
    P = pkg()
    st = _dense_strides(fmt, m, n, k)
    assert P.typed_plan(fmt, m, n, k, 128, st) == expect == P.plan(fmt, m, n, k, 128)
    assert P.typed_plan(fmt, m, n, k, 128, st, aligned16=False) == "strided"
    for i, bad in ((0, k + 8), (1, 2), (2, st[2] + 1), (5, 2), (6, st[6] + 3), (8, n + 8)):
        if i in (0, 8) and m == 1:
            continue                    # a single row's stride is never used
        s2 = list(st)
        s2[i] = bad
        assert P.typed_plan(fmt, m, n, k, 128, s2) == "strided", (i, bad)
    assert P.typed_plan(fmt, m, n, k + 64, 128, _dense_strides(fmt, m, n, k + 64)) == "strided"


def test_init_without_device_reports_backend_disabled():
    import torch
    P = pkg()
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    assert P.lib().w4a16_init(0) == P.ERR_BACKEND_DISABLED


def test_act_order_argument_errors():
    P = pkg()
    L = P.lib()
    v = ctypes.c_void_p(256)
    w = ctypes.c_void_p(512)
    assert L.w4a16_prepare_act_order(None, P.FMT_AWQ, v, v, 4096, 512, 128, w, w) == P.ERR_INVALID_ARG
    assert L.w4a16_prepare_act_order(None, P.FMT_GPTQ, v, v, 4096, 512, 128, v, w) == P.ERR_INVALID_ARG
    assert "alias" in L.w4a16_last_error().decode()
    assert L.w4a16_prepare_act_order(None, P.FMT_GPTQ, v, v, 4000, 512, 128, w, w) == P.ERR_INVALID_ARG
    assert L.w4a16_gemm_act_order(None, P.FMT_AWQ, v, v, v, v, v, v, 1, 512, 4096, 128, 1) == P.ERR_INVALID_ARG
    assert L.w4a16_gemm_act_order(None, P.FMT_GPTQ, v, v, v, v, None, v, 1, 512, 4096, 128, 1) == P.ERR_INVALID_ARG
    assert "perm" in L.w4a16_last_error().decode()


# ------------------------------------------------------------------ prepared layout

def test_prepared_bytes_matches_the_layout():
    """w4a16_prepared_bytes equals the strip size of the layout's restatement (tests/synth.py)
    times the strip count, and is 0 for shapes the layout does not take."""
    from synth import prepared_strip_bytes
    P = pkg()
    for K, N, G in ((4096, 14336, 128), (14336, 4096, 128), (4096, 4096, 128), (1024, 64, 32),
                    (2048, 16, 64), (4096, 32, 256), (4096, 48, 4096)):
        assert P.prepared_bytes(K, N, G) == N // 16 * prepared_strip_bytes(K, G), (K, N, G)
    for K, N, G in ((4096, 4104, 128), (4000, 4096, 125), (4096, 4096, 96), (4096, 4096, 16),
                    (65536, 16, 128), (0, 16, 128)):
        assert P.prepared_bytes(K, N, G) == 0, (K, N, G)


@pytest.mark.parametrize("over,code,needle", [
    (dict(N=4104), 2, "N % 16"),
    (dict(G=96, K=3072), 2, "group_size 32, 64"),
    (dict(K=4000, G=125), 2, "K % 128"),
    (dict(nbytes=1024), 1, "too small"),
    (dict(buf=4096 + 16), 1, "256-byte aligned"),
    (dict(qw=None), 1, "null pointer"),
    (dict(fmt=2, zo=-3), 0, None),          # the AWQ format ignores the GPTQ zero offset
    (dict(fmt=0, zo=17), 1, "gptq_zero_offset"),
])
def test_prepare_layout_argument_errors(over, code, needle):
    P = pkg()
    a = dict(fmt=P.FMT_AWQ, qw=1 << 20, sc=2 << 20, qz=3 << 20, K=4096, N=4096, G=128, zo=0,
             buf=1 << 30, nbytes=1 << 30)
    a.update(over)
    if code == 0:
        return   # a valid request would launch kernels: not here
    p = lambda v: None if v is None else ctypes.c_void_p(v)
    rc = P.lib().w4a16_prepare_layout(None, a["fmt"], p(a["qw"]), p(a["sc"]), p(a["qz"]), a["K"],
                                      a["N"], a["G"], a["zo"], p(a["buf"]), a["nbytes"])
    assert rc == code
    assert needle in P.lib().w4a16_last_error().decode()


def test_prepare_layout_rejects_overlap():
    P = pkg()
    K, N, G = 4096, 4096, 128
    base = 1 << 30
    rc = P.lib().w4a16_prepare_layout(None, P.FMT_AWQ, ctypes.c_void_p(base), ctypes.c_void_p(2 << 30),
                                      ctypes.c_void_p(3 << 30), K, N, G, 0, ctypes.c_void_p(base + 256),
                                      P.prepared_bytes(K, N, G))
    assert rc == P.ERR_INVALID_ARG and "overlap" in P.lib().w4a16_last_error().decode()


@pytest.mark.parametrize("M,N,K,G,code,needle", [
    (0, 4096, 4096, 128, 1, "M (0)"),
    (1, 4100, 4096, 128, 2, "N % 16"),
    (1, 4096, 3072, 48, 2, "group_size"),
])
def test_gemm_prepared_argument_errors(M, N, K, G, code, needle):
    P = pkg()
    rc = P.lib().w4a16_gemm_prepared(None, ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 30), None,
                                     ctypes.c_void_p(2 << 20), M, N, K, G)
    assert rc == code
    assert needle in P.lib().w4a16_last_error().decode()


@pytest.mark.parametrize("M,N,K,G,gi,code,needle", [
    (0, 4096, 4096, 128, 3 << 20, 1, "M (0)"),
    (1, 4100, 4096, 128, 3 << 20, 2, "N % 16"),
    (1, 4096, 3072, 48, 3 << 20, 2, "group_size"),
    (16, 4096, 4096, 128, None, 1, "null pointer"),
    (16, 4096, 4096, 128, (3 << 20) + 4, 1, "g_idx must be 16-byte aligned"),
])
def test_gemm_prepared_gidx_argument_errors(M, N, K, G, gi, code, needle):
    """w4a16_gemm_prepared_gidx checks its shape, pointers and alignment before any HIP call."""
    P = pkg()
    rc = P.lib().w4a16_gemm_prepared_gidx(None, ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 30),
                                          None if gi is None else ctypes.c_void_p(gi),
                                          ctypes.c_void_p(2 << 20), M, N, K, G)
    assert rc == code
    assert needle in P.lib().w4a16_last_error().decode()


def test_gemm_prepared_python_refuses_perm_with_g_idx():
    """gemm_prepared takes either the group-order permutation or g_idx, never both (checked
    before any device access)."""
    import torch
    P = pkg()
    w = P.PreparedWeights(torch.empty(0, dtype=torch.uint8), 4096, 4096, 128)
    x = torch.empty((4, 4096), dtype=torch.float16)
    i = torch.empty(4096, dtype=torch.int32)
    with pytest.raises(P.InvalidArgument, match="not both"):
        P.gemm_prepared(x, w, perm=i, g_idx=i)
