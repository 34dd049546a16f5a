import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


def pytest_sessionfinish(session, exitstatus):
    mod = sys.modules.get("tests.hip_helpers")
    if mod is not None:
        mod.write_margins(REPO)


def relerr(a, b):
    """||a-b|| / ||b|| (the reference tests' metric, test_k1_k9.py:48-49)."""
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).norm() / (b.norm() + 1e-30)).item()


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(REPO, "tests", "golden", "dm_golden.npz")
    return dict(np.load(path))
