import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libkandle_hip.so on the device)")


@pytest.fixture(scope="session")
def hip():
    """The HIP backend on device 0 (created once per session)."""
    from kandle_amd import HipBackend, env

    try:
        return env.get_backend("hip")
    except RuntimeError:
        return HipBackend.create(0)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a fault leaves the test id in the output.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
