"""Shared pytest setup: the `gpu` marker, import paths, and parity helpers."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "inference-agent_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

# Parity bar from BASELINE.json north_star: max|d| <= 2e-3 and relative L2 <= 1e-3 in f32.
MAX_ABS_TOL = 2e-3
REL_L2_TOL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def ensure_built(target: str) -> None:
    """Builds liboracle.so or libingot_attn.so in-tree if missing (no GPU needed)."""
    if target == "oracle":
        if not os.path.exists(os.path.join(ORACLE, "liboracle.so")):
            subprocess.run(["make", "-C", ORACLE], check=True, capture_output=True)
    elif target == "lib":
        if not os.path.exists(os.path.join(PKG, "libingot_attn.so")):
            subprocess.run(["make", "-C", PKG, "-j4"], check=True, capture_output=True)


def parity(got: np.ndarray, want: np.ndarray):
    """Returns (max_abs, rel_l2) of got vs want, in float64."""
    got = np.asarray(got, dtype=np.float64).ravel()
    want = np.asarray(want, dtype=np.float64).ravel()
    assert np.all(np.isfinite(got)), "non-finite output"
    d = got - want
    max_abs = float(np.max(np.abs(d))) if d.size else 0.0
    den = float(np.linalg.norm(want))
    rel = float(np.linalg.norm(d) / den) if den > 0 else float(np.linalg.norm(d))
    return max_abs, rel


def assert_parity(got, want, what=""):
    max_abs, rel = parity(got, want)
    assert max_abs <= MAX_ABS_TOL and rel <= REL_L2_TOL, (
        f"{what}: max|d|={max_abs:.3e} (tol {MAX_ABS_TOL}), rel-L2={rel:.3e} (tol {REL_L2_TOL})")
    return max_abs, rel


@pytest.fixture(scope="session")
def oracle_mod():
    ensure_built("oracle")
    import oracle_lib as oracle

    return oracle
