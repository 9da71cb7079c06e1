import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through libsile_hip")


@pytest.fixture(scope="session")
def hip():
    """Initialises device 0 through the C ABI and returns the binding module."""
    from sile_amd import _abi
    _abi.init(0)
    return _abi
