import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libprana_hip.so")
    config.addinivalue_line("markers", "slow: long-running (minutes)")


def _stamp(msg):
    sys.stdout.write(msg + "\n")
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # Print the case before any GPU work so a lost box still names it.
    if request.node.get_closest_marker("gpu"):
        _stamp(f"[gpu-case] {request.node.nodeid}")
    yield
