"""Shared test helpers: package loading, device transfer and the parity tolerance."""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

RTOL = 1e-2  # the path's bar: max relative error 1e-2 vs fp32 dequant-then-matmul


def pkg():
    return __graft_entry__.load_package()


def to_dev(a, device="cuda:0"):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(device)


def rel_err(got, ref) -> float:
    """max |got - ref| / max(|ref|, rms(ref)) -- relative error with an rms floor.

    A pure per-element relative error is unbounded where the reference is ~0; the floor
    (the reference's own rms) follows the reference's tol = max(atol, rel*|want|) pattern
    (crates/triton-runtime/examples/run_vec_add.rs:142)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    floor = np.sqrt(np.mean(ref ** 2)) if ref.size else 0.0
    scale = np.maximum(np.abs(ref), floor)
    scale[scale == 0] = 1.0
    return float(np.max(np.abs(got - ref) / scale)) if ref.size else 0.0


def assert_parity(got, ref, tol=RTOL, what=""):
    e = rel_err(got, ref)
    assert e <= tol, f"{what}: max relative error {e:.3e} > {tol}"
    return e
