import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    """The library context on device 0 (GPU tests only)."""
    from p0pc0rn_amd import capi
    capi.open_device(0)
    info = capi.device_info()
    print("device:", info, flush=True)
    yield capi
    capi.done()


def rel_l2(got, want):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def cos_sim(got, want):
    """engine/kcheck.js compare(): cosine similarity"""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(got @ want / max(np.sqrt((got @ got) * (want @ want)), 1e-30))
