import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    """A vtb_hip context on cuda:0.  Skips only where no GPU device node
    exists at all; on a GPU box a failing init is an error, never a skip."""
    if not os.path.exists("/dev/kfd"):
        pytest.skip("no GPU (/dev/kfd absent)")
    import vantablack_amd as vb
    c = vb.Context()
    yield c
    c.close()
