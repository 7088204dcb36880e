"""The Rust DeviceRuntime backend's C call sequence on the GPU: tests/native/replay_hiprt (built
by __graft_entry__.build()) issues the hiprt_* calls rust/triton-runtime-hip makes for
HipRuntime::new, load_module, launch of awq_gemm_int4_typed with the reference's 19
parameters + 2 scratch pointers, and the copies back; its output must match the oracle and
w4a16_gemm's. Runs as a child process (the test process only reads files)."""
import os
import subprocess

import numpy as np
import pytest

from helpers import ROOT, assert_parity, pkg, to_dev
from synth import Problem

pytestmark = pytest.mark.gpu
AWQ = 2
REPLAY = os.path.join(ROOT, "tests", "native", "_build", "replay_hiprt")


@pytest.mark.parametrize("M,K,N,G", [(5, 256, 128, 128), (70, 512, 200 // 8 * 8, 64)])
def test_rust_backend_call_sequence_replay(tmp_path, orc, M, K, N, G):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(REPLAY), "tests/native/_build/replay_hiprt missing: run __graft_entry__.build()"
    P = pkg()
    p = Problem(AWQ, M=M, K=K, N=N, G=G, seed=7700 + M)
    inp = tmp_path / "in.bin"
    out = tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(np.array([M, N, K, G], dtype=np.int32).tobytes())
        for a in (p.x, p.qweight, p.scales, p.qzeros):
            f.write(np.ascontiguousarray(a).tobytes())
    print(f"replay M={M} K={K} N={N} G={G}", flush=True)
    r = subprocess.run(["timeout", "-k", "10", "120", REPLAY, P.HSACO_PATH, str(inp), str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    y = np.fromfile(out, dtype=np.float16).reshape(M, N)
    ref = orc.w4a16_gemm(AWQ, p.x, p.qweight, p.scales, p.qzeros, K, N, G, want_f32=True)[1]
    assert_parity(y, ref, what=f"replayed launch M={M}")
    # the same problem through the op-level entry point: both are within the bar of the oracle
    y_op = P.gemm(to_dev(p.x), to_dev(p.qweight), to_dev(p.scales), to_dev(p.qzeros), fmt="awq",
                  group_size=G).cpu().numpy()
    assert_parity(y, y_op.astype(np.float64), what="replay vs w4a16_gemm")
