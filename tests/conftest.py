import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(autouse=True)
def fresh_program():
    """Every test traces into a fresh global context (the reference runs its
    tests with process isolation for the same reason)."""
    import ad_amd
    ad_amd.reset()
    yield
    ad_amd.reset()


_HIP_DEVICE = {}


@pytest.fixture
def hip():
    """A fresh HIPDevice per program (one context per test)."""
    from ad_amd.device.hip import HIPDevice
    devs = []

    def make(**kw):
        d = HIPDevice(**kw)
        devs.append(d)
        return d
    yield make
    for d in devs:
        d.close()
