"""CPU checks of the host logic behind the XCD-local split merge: the
decode launcher runs every split of a unit on one XCD only when vtb_hip_init
saw workgroups dealt over the XCDs round-robin (workgroup i on the XCD of
workgroup i mod nx).  vtb_hip_xcd_deal is that check; these cases exercise
it on XCC-id patterns without a GPU."""
import ctypes

import numpy as np
import pytest


@pytest.fixture(scope="module")
def deal():
    from vantablack_amd import hip
    L = hip.lib()

    def f(ids):
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        return int(L.vtb_hip_xcd_deal(a.ctypes.data_as(ctypes.c_void_p), len(a)))
    return f


def test_round_robin_from_any_start(deal):
    n = 4096
    for nx in (8, 4, 2):
        for r in range(nx):
            assert deal((np.arange(n) + r) % nx) == nx
    # XCC ids need not be 0..nx-1 in order, only distinct and periodic.
    perm = np.array([3, 0, 7, 1, 6, 2, 5, 4])
    assert deal(perm[np.arange(n) % 8]) == 8


def test_one_xcd(deal):
    assert deal(np.full(4096, 5)) == 1


def test_other_dealings_are_refused(deal):
    n = 4096
    i = np.arange(n)
    assert deal((i // 2) % 8) == 0          # pairs of workgroups per XCD
    assert deal((i // 32) % 8) == 0         # blocks of workgroups per XCD
    ids = i % 8
    ids[1000] = (ids[1000] + 1) % 8         # one workgroup off its XCD
    assert deal(ids) == 0
    rng = np.random.default_rng(0)
    assert deal(rng.integers(0, 8, n)) == 0


def test_degenerate_inputs(deal):
    assert deal(np.arange(8)) == 0          # no repeat seen
    assert deal(np.array([0, 1, -1, 0, 1, -1])) == 0
    assert deal(np.array([16, 16, 16, 16])) == 0
    assert deal(np.array([], dtype=np.int32)) == 0
