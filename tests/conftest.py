import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long CPU test")


def pytest_sessionstart(session):
    """A tree without the native libraries (built artefacts are not in git)
    builds them once first; a built tree is used as it is."""
    import __graft_entry__

    __graft_entry__.ensure_built()


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as o

    o.lib()
    return o
