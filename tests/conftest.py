import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "seedvr2-ncnn_amd", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through the C ABI; fails loudly if there is none."""
    import awa_hip

    if awa_hip.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests must run on an MI355X")
    awa_hip.init(0)
    return awa_hip
