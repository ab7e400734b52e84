"""pytest configuration: the `gpu` marker, the repository root on sys.path (for `kvtier` and `oracle`)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkvtier.so")


@pytest.fixture(scope="session")
def kvt_pkg():
    import kvtier  # noqa: F401  (loads the package directory)
    return kvtier
