import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "recipe-dev_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through librqmv; a gpu-marked test fails loudly
    (never falls back) when the library or the device is missing."""
    import rqmv

    if rqmv.device_count() < 1:
        pytest.fail("no HIP device visible")
    rqmv.init(0)
    return rqmv
