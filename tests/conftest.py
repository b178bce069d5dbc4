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


# Split workspace bound to the session stream: enough for every split the
# GPU tests run or pin (16 K chunks of a 2048 x 2048 f32 output at most).
STREAM_WORKSPACE = 256 << 20


@pytest.fixture(scope="session")
def stream(px_gpu):
    s = px_gpu.Stream()
    px_gpu.bind_workspace(s, STREAM_WORKSPACE)
    return s
