"""CPU checks through native test programs (tests/native/): the oracle and the C-ABI op layer
(argument validation, kernel planning over a sweep of shapes) built with AddressSanitizer and
UndefinedBehaviorSanitizer. No GPU work: every call either fails validation before any HIP
call or only plans."""
import os
import subprocess

import pytest

from helpers import ROOT

NATIVE = os.path.join(ROOT, "tests", "native")


def _build(target):
    r = subprocess.run(["make", "-C", NATIVE, target], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return os.path.join(NATIVE, target)


def _run_sanitized(path):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([path], capture_output=True, text=True, timeout=600, env=env)
    report = r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in report, report[-4000:]
    assert "runtime error" not in report, report[-4000:]
    assert r.returncode == 0, report[-4000:]
    return r.stdout


def test_oracle_under_sanitizers():
    out = _run_sanitized(_build("_build/orc_selftest"))
    assert "all checks passed" in out


def test_c_abi_validation_under_sanitizers():
    if not os.path.exists(os.path.join(ROOT, "triton-rs_amd", "_build", "kernels_gemv.o")):
        pytest.fail("kernel objects missing: run __graft_entry__.build() first")
    out = _run_sanitized(_build("_build/abi_selftest"))
    assert "all checks passed" in out
