import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def ctx():
    from edgerunner_amd import Context
    c = Context(int(os.environ.get("ER_DEVICE", "0")))
    yield c


@pytest.fixture(scope="session")
def gemv(ctx):
    from edgerunner_amd import GEMVKernel
    return GEMVKernel(ctx)


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a crash is attributable
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
