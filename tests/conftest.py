import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libfrq.so on the device)")


@pytest.fixture(scope="session")
def ctx():
    """A libfrq context on device 0.  GPU tests fail (not skip) when the
    library or the device is missing: there is no fallback path."""
    import fieldrun_amd as fa
    c = fa.Context(0)
    yield c
    c.close()
