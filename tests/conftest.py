import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "phobos-lang_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def px_gpu():
    """Initialises the HIP backend on device 0 (fails loudly without a GPU)."""
    import phobos_amd as px
    px.init(0)
    return px


@pytest.fixture(scope="session")
def stream(px_gpu):
    return px_gpu.Stream()
