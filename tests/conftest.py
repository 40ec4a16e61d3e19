import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through libneedle_hip.so")


@pytest.fixture(scope="session")
def orc():
    """The oracle library (built on first use)."""
    from oracle import oracle as O
    return O


@pytest.fixture(scope="session")
def hip():
    """The product library, initialised on device 0.  Fails (never skips) when
    the library or the device is missing: GPU tests must run the HIP path."""
    import needle_cs_amd as N
    N.check(N.lib().nhip_init(0))
    return N
