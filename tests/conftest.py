import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def ctx():
    """One device context for every GPU test of the session."""
    from voxgen_amd.runtime import Context
    c = Context(int(os.environ.get("VOXHIP_DEVICE", "0")))
    yield c
    c.close()


def rel_l2(a, b) -> float:
    import numpy as np
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
