import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libfa_hip.so")


@pytest.fixture(scope="session")
def library_path():
    """Path of the built C-ABI library; builds it (content-hashed) when absent."""
    from fa_amd import build

    if not build.up_to_date():
        build.build()
    return str(build.LIBRARY)
