"""Build the gfx950 W4A16 library in-tree.

Outputs (next to this file):
  libw4a16.so         C ABI of include/w4a16.h (kernels embedded as a gfx950 fat binary)
  w4a16_typed.hsaco   code object with the reference-named kernels, for hiprt_module_load
  w4a16_typed.json    launch metadata for that code object

Every HIP compile line carries `-Xclang -target-feature -Xclang -packed-fp32-ops`, which
turns off packed-fp32 instruction selection on this target.
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libw4a16.so")
HSACO = os.path.join(HERE, "w4a16_typed.hsaco")
META = os.path.join(HERE, "w4a16_typed.json")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]

SOURCES = ["api.cpp", "hiprt.cpp", "kernels_gemv.hip", "kernels_prefill.hip", "kernels_skinny.hip", "kernels_strided.hip", "kernels_moe.hip", "act_order.hip", "noalloc.hip", "prepared.hip"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is noise
    err = "\n".join(l for l in r.stderr.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l
                    and "unused during compilation" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    # .cpp sources are host code only (no device pass for a default target)
    lang = ["-x", "hip", f"--offload-arch={ARCH}"] if src.endswith(".hip") else ["--cuda-host-only"]
    _run([HIPCC, *lang, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
        fut_hsaco = ex.submit(_run, [HIPCC, "-x", "hip", f"--offload-arch={ARCH}", *COMMON,
                                     "--genco", "--no-gpu-bundle-output", os.path.join(CSRC, "typed_module.hip"),
                                     "-o", HSACO + ".tmp"])
        fut_hsaco.result()
    os.replace(HSACO + ".tmp", HSACO)
    _run([HIPCC, "-shared", "-fPIC", *objs, "-o", LIB + ".tmp"])
    os.replace(LIB + ".tmp", LIB)
    meta = {
        "kernels": [
            {"name": name, "num_warps": 8, "threads_per_block": 256, "warp_size": 64,
             "shared_mem": 0, "global_scratch_size": 0, "profile_scratch_size": 0,
             "block_m": 64, "block_n": 64, "grid": "[cdiv(m, 64), cdiv(n, 64), 1]",
             "params": 21}
            for name in ("w4a16_gptq_gemm_typed", "awq_gemm_int4_typed")
        ],
        "target": f"amdgcn-amd-amdhsa--{ARCH}",
    }
    with open(META, "w") as f:
        json.dump(meta, f, indent=2)
    if verbose:
        print(f"built {LIB} and {HSACO}")
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    for p in (LIB, HSACO, META):
        if os.path.exists(p):
            os.remove(p)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build()
