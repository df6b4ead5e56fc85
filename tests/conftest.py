"""Shared test plumbing: the `gpu` marker, the oracle import, device buffers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle", "_build")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    import cptc_oracle  # CPU oracle: the checker (test infrastructure)
    return cptc_oracle


@pytest.fixture(scope="session")
def ca():
    import cptc_amd
    return cptc_amd


@pytest.fixture(scope="session")
def dev(ca):
    """Device 0 through libcptc's own HIP runtime (device buffers are
    cptc_amd.DevBuf; no second HIP runtime is loaded into the process)."""
    assert ca.device_count() >= 1, "GPU test run without a visible HIP device"
    return ca


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
