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


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Downstream-argmax agreement of every f16/bf16 parity case that ran:
    rows checked and rows whose argmax differed by a near tie (accepted by
    tests.parity.check only within TIE_REL of the best logit)."""
    try:
        from tests import parity
    except ImportError:
        return
    if not parity.FLIPS:
        return
    tr = terminalreporter
    n_cases = len(parity.FLIPS)
    flipped = [(w, n, k) for w, n, k in parity.FLIPS if k]
    tr.write_sep("-", f"downstream argmax: {n_cases} f16/bf16 cases, "
                      f"{sum(n for _, n, _ in parity.FLIPS)} rows, {len(flipped)} cases with near-tie flips")
    for w, n, k in flipped:
        tr.write_line(f"  tie-flip: {w}: {k} of {n} rows")
