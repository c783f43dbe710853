"""Shared test setup.

Markers: `gpu` tests need an MI355X (they run through the C ABI on cuda:0);
everything else runs on the CPU.  The oracle (oracle/, the C restatement of
tools/ref_qwen3.py) is used here only as the checker.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "qwen3-tile-ops_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def golden(name: str):
    path = GOLDEN / name
    if name.endswith(".json"):
        return json.loads(path.read_text())
    return np.load(path, allow_pickle=False)


@pytest.fixture(scope="session")
def gold_meta():
    return golden("meta.json")


@pytest.fixture(scope="session")
def cuda():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a ROCm device (cuda:0)"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.shape != b.shape:
        return False
    if a.dtype == np.float32:
        return bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))
    return bool(np.array_equal(a, b))


def describe_diff(a: np.ndarray, b: np.ndarray) -> str:
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape:
        return f"shape {a.shape} != {b.shape}"
    if np.issubdtype(a.dtype, np.integer):
        d = a.astype(np.int64) - b.astype(np.int64)
        bad = np.flatnonzero(d)
        return f"{bad.size}/{a.size} int mismatches; first @{bad[:5].tolist()}"
    ua, ub = a.view(np.uint32).ravel(), b.view(np.uint32).ravel()
    bad = np.flatnonzero(ua != ub)
    if bad.size == 0:
        return "bit-exact"
    i = bad[0]
    return (f"{bad.size}/{a.size} f32 bit mismatches; first @{i}: {a.ravel()[i]!r} vs "
            f"{b.ravel()[i]!r}; max|d|={np.nanmax(np.abs(a.astype(np.float64) - b)):.3g}")
