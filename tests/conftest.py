"""Shared test setup.

* registers the `gpu` marker (tests that need an MI355X);
* puts the host package (acestep.cpp_amd/, module `mxfa`) and the CPU oracle
  (oracle/, module `oracle`) on sys.path;
* small helpers: parity metrics with the definitions of the reference's
  src/debug.h:107-131 (cosine, max-abs) applied per output row.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "acestep.cpp_amd")
ORACLE = os.path.join(REPO, "oracle")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)

# Parity bar of the benchmark (fp32 accumulate).
MAX_ABS_TOL = 2e-3
ROW_COS_TOL = 0.9999


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


def row_metrics(got: np.ndarray, ref: np.ndarray) -> dict:
    """max-abs over all elements and the minimum per-row cosine, rows = last
    axis (one output row of D values per (batch, query, head)).  A row that
    is zero in both is a perfect match (fully masked rows)."""
    g = np.asarray(got, dtype=np.float64).reshape(-1, got.shape[-1])
    r = np.asarray(ref, dtype=np.float64).reshape(-1, ref.shape[-1])
    max_abs = float(np.max(np.abs(g - r))) if g.size else 0.0
    dot = np.sum(g * r, axis=1)
    ng = np.sqrt(np.sum(g * g, axis=1))
    nr = np.sqrt(np.sum(r * r, axis=1))
    both_zero = (ng < 1e-30) & (nr < 1e-30)
    with np.errstate(invalid="ignore", divide="ignore"):
        cos = np.where(both_zero, 1.0, np.where((ng < 1e-30) | (nr < 1e-30), 0.0, dot / (ng * nr)))
    return dict(max_abs=max_abs, min_cos=float(np.min(cos)) if cos.size else 1.0,
                mean_cos=float(np.mean(cos)) if cos.size else 1.0,
                nan=bool(np.isnan(g).any()))


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle
