import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "nexus-inference-engine-_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def ctx():
    """One nx_ctx for the whole GPU session (tests run in one process)."""
    import nexus_amd
    c = nexus_amd.Context(0)
    print(f"[gpu] device: {c.device_name()}", flush=True)
    yield c
    c.close()


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the tolerance metric of the parity tests)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - ref)) / denom)


def f16(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)
