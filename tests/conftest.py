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
    """Path of the built C-ABI library; builds it (content-hashed) when absent.
    ``FA_TEST_LIBRARY`` names another build of it to test instead (e.g. the
    host-sanitizer build, ``python -m fa_amd.build --sanitize``)."""
    from fa_amd import build

    other = os.environ.get("FA_TEST_LIBRARY")
    if other:
        return other
    if not build.up_to_date():
        build.build()
    return str(build.LIBRARY)
