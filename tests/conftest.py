import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for all GPU tests (the reference shares one MetalContext)."""
    from runit_mac_amd import dispatch as d
    c = d.HipContext()
    yield c
    c.close()


@pytest.fixture(scope="session")
def ora():
    import oracle_lib
    return oracle_lib
