"""pytest setup: the `gpu` marker, import paths, and shared helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libdaiza_hip.so")


def normwise_rel(a, b):
    """max|a-b| / max|b| — the per-vector relative error used for the 1e-3 bar."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / (d if d > 0 else 1.0))


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def dz():
    """The HIP library, initialised on device 0 (gpu tests only)."""
    import daiza_amd
    L = daiza_amd.lib()
    rc = L.dz_device_init(0)
    if rc != 0:
        raise RuntimeError("dz_device_init failed: " + L.dz_last_error().decode())
    return daiza_amd
