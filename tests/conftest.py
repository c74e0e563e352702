import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    o = oracle()
    o.set_threads(8)
    return o


@pytest.fixture(scope="session")
def gpu():
    """Initialise device 0. GPU tests fail loudly (never skip) without one."""
    from peregrine_amd import device

    n = device.device_count()
    assert n >= 1, "no HIP device visible; GPU tests need an MI355X"
    device.init(0)
    print(f"[gpu] {device.device_name()}", flush=True)
    return device


@pytest.fixture
def rng():
    return np.random.default_rng(0)
