"""CPU checks of bench.py's contract: the algorithmic byte counts its GB/s figures divide by
(each configuration's qweight, scales, qzeros, g_idx, x and out, each counted once) and the
refusal of a multi-GPU run, which this single-GPU build does not measure."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402  (imports no GPU code at module level)


@pytest.mark.parametrize("fmt,M,K,N,act_order,expect", [
    ("gptq_sym", 1, 4096, 4096, False, 8_667_136),      # config 0
    ("awq", 1, 4096, 14336, False, 30_543_872),         # config 1 (both shapes)
    ("awq", 1, 14336, 4096, False, 30_543_872),
    ("awq", 4, 4096, 14336, False, 30_654_464),
    ("awq", 8, 14336, 4096, False, 30_801_920),
    ("gptq", 16, 4096, 6144, True, 13_418_496),          # config 2, act-order
    ("gptq", 32, 4096, 6144, True, 13_746_176),
    ("gptq", 64, 4096, 6144, True, 14_401_536),
    ("awq", 2048, 4096, 14336, False, 106_004_480),     # config 3
])
def test_algorithmic_bytes_match_the_per_config_table(fmt, M, K, N, act_order, expect):
    """The per-configuration totals are the scope table's figures, written down from the
    tensor sizes (e.g. config 2 at M=16: 12,582,912 + 393,216 + 98,304 + 16,384 + 131,072 +
    196,608)."""
    assert bench.algorithmic_bytes(fmt, M, K, N, 128, act_order) == expect


def test_multi_gpu_run_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)
