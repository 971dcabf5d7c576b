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


class DeviceBankView:
    """The oracle's view of a device ``ResidentBank``: ``dequant(e, role)`` copies
    one expert role to the host and decodes it with the oracle's format code.

    ``prefetch(experts)`` starts decoding those experts' roles, in the order the
    oracle layer asks for them (ascending expert, w1, w3, w2), on a thread pool
    that stays at most ``window`` roles ahead; each prefetched role is handed
    out once and then dropped, so a layer of hundreds of experts never holds
    more than the window in host memory.
    """

    def __init__(self, bank, workers: int = 8, window: int = 48):
        import concurrent.futures as cf
        self.bank, self.quant = bank, bank.quant
        self._pool = cf.ThreadPoolExecutor(max_workers=workers)
        self._window = window
        self._order: list = []
        self._next = 0
        self._ready: dict = {}

    def _load(self, e: int, role: str):
        from oracle import formats as F
        parts = [t[e].cpu().numpy() for t in self.bank.roles[role]]
        return F.fp4_dequant(*parts) if self.quant == "fp4" else F.q3_dequant(*parts)

    def prefetch(self, experts) -> "DeviceBankView":
        self._order = [(int(e), r) for e in sorted(set(int(v) for v in experts)) for r in ("w1", "w3", "w2")]
        self._next = 0
        self._ready.clear()
        self._top_up()
        return self

    def _top_up(self) -> None:
        while self._next < len(self._order) and len(self._ready) < self._window:
            key = self._order[self._next]
            self._next += 1
            self._ready[key] = self._pool.submit(self._load, *key)

    def dequant(self, e, role):
        fut = self._ready.pop((int(e), role), None)
        self._top_up()
        return fut.result() if fut is not None else self._load(int(e), role)

    def close(self) -> None:
        self._pool.shutdown(wait=True)
