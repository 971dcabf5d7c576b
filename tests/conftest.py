"""pytest configuration: import paths, the ``gpu`` marker, shared helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "deepseeker-v4.1_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for p in (str(ROOT), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libdsk_moe.so")


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def assert_layer_close(got, ref, cos_min=0.99999, rel_max=1e-2):
    """Output tolerance of the layer: cosine >= 0.99999 and
    max|got - ref| / max|ref| <= 1e-2 (ref = the oracle's float32 output)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    c = cosine(g, r)
    rel = float(np.abs(g - r).max() / max(np.abs(r).max(), 1e-30))
    assert c >= cos_min and rel <= rel_max, f"cos={c:.8f} rel={rel:.3e}"
    return c, rel


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(GOLDEN / name, allow_pickle=False)
    return load
