"""Shared test setup.

GPU tests (marked ``gpu``) run the HIP path through the C ABI and compare it
with the CPU oracle (oracle/, test infrastructure only) on the same seeded
inputs.  CPU tests (``-m "not gpu"``) pin the oracle itself and check the
host-side logic and the library's exported symbols without touching a GPU.
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    if not os.path.exists(o.LIB_PATH):
        o.build()
    return o


@pytest.fixture(scope="session")
def kat():
    return dict(np.load(os.path.join(REPO, "tests", "golden", "kat.npz")))


@pytest.fixture(scope="session")
def backend():
    from realm_amd.backend import HipGpuBackend
    return HipGpuBackend(0)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
