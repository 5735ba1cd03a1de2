# SPDX-License-Identifier: Apache-2.0
"""Shared test setup: import paths, the `gpu` marker, fixture loading."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "kimi-k3-in-c_amd", REPO / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"
REF_OPS = GOLDEN / "ref_ops"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_fixture(name: str) -> dict:
    """A reference op fixture: every {"shape", "data"} entry becomes a float32 array."""
    raw = json.loads((REF_OPS / f"{name}.json").read_text())
    out = {}
    for k, v in raw.items():
        if isinstance(v, dict) and "data" in v:
            out[k] = np.asarray(v["data"], dtype=np.float32).reshape(v.get("shape", [-1]))
        else:
            out[k] = v
    return out


def manifest_tol() -> tuple[float, float]:
    """(atol, rtol) from the fixture manifest, the reference's pass criterion."""
    m = json.loads((REF_OPS / "MANIFEST.json").read_text())["tolerance"]
    return float(m["fp32_abs"]), float(m["fp32_rel"])


def worst_ratio(got, want, atol: float, rtol: float) -> float:
    """max |got - want| / (atol + rtol |want|): the reference comparator
    (tests/unit/test_ops.c:114-128); <= 1 passes."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.size == 0:
        return 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(np.max(np.abs(got - want) / (atol + rtol * np.abs(want))))


def assert_close(got, want, atol: float, rtol: float, what: str = "") -> float:
    r = worst_ratio(got, want, atol, rtol)
    assert r <= 1.0, f"{what}: worst {r:.3f}x tolerance (atol={atol:g}, rtol={rtol:g})"
    return r


@pytest.fixture(scope="session")
def gpu():
    """The HIP library with a visible device; GPU tests fail (not skip) without one."""
    import torch
    import k3kda
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    L = k3kda.lib()
    assert L.k3hip_device_count() >= 1
    return k3kda
