"""The GPU parity check itself (tests/parity.py), exercised on the CPU: it must
pass an exact match, reject a wrong output that stays numerically close, reject
a real argmax change, and accept only near-tie flips, at most 1% of rows."""
import numpy as np
import pytest

from tests import parity
from tests.parity import TIE_REL, argmax_mismatches, check, downstream_logits


@pytest.fixture(autouse=True)
def _no_flip_records():
    """The planted ties here are not parity results: drop their FLIPS records."""
    n = len(parity.FLIPS)
    yield
    del parity.FLIPS[n:]


def _ref(orc, n_rows=200, n_heads=4, d=32, seed=3):
    return orc.normal(seed, n_rows * n_heads * d).reshape(n_rows, n_heads * d)


def test_exact_match_passes(orc):
    ref = _ref(orc)
    check(orc, ref.copy(), ref, 4, "bf16", n_queries=ref.shape[0], what="exact")


def test_relative_error_above_tolerance_fails(orc):
    ref = _ref(orc)
    got = ref * np.float32(1.003)
    with pytest.raises(AssertionError, match="rel err"):
        check(orc, got, ref, 4, "bf16", n_queries=ref.shape[0], what="scaled")


def test_real_argmax_change_fails(orc):
    # Row r's two best reference logits are set 3x the tie threshold apart;
    # `got` crosses them with an output change far inside the 2e-3 relative
    # tolerance, so only the argmax rule can catch it.
    ref = _ref(orc).astype(np.float64)
    n = ref.shape[0]
    W = orc.normal(777, 2048 * ref.shape[1]).astype(np.float64).reshape(2048, -1)
    r = 5
    l = W @ ref[r]
    best, other = int(l.argmax()), int(np.argsort(l)[-2])
    dvec = W[other] - W[best]
    scale = np.max(np.abs(l))
    target_gap = 3 * TIE_REL * scale
    ref[r] += dvec * ((l[best] - l[other] - target_gap) / float(dvec @ dvec))
    got = ref.copy()
    got[r] += dvec * (1.2 * target_gap / float(dvec @ dvec))
    ref32, got32 = ref.astype(np.float32), got.astype(np.float32)
    rows, not_tie = argmax_mismatches(orc, got32, ref32, n)
    assert list(rows) == [r] and not_tie == [r]
    with pytest.raises(AssertionError, match="argmax differs"):
        check(orc, got32, ref32, 4, "bf16", n_queries=n, what="moved")


def test_near_tie_flip_is_accepted_but_capped(orc):
    ref = _ref(orc).astype(np.float64)
    n = ref.shape[0]
    W = orc.normal(777, 2048 * ref.shape[1]).astype(np.float64).reshape(2048, -1)

    def make_tie(x, r):
        # Nudge row r so its two best logits are equal; return the direction
        # that moves logit `other` up against `best` (unit logit change per
        # unit step) and the row's logit scale.
        l = W @ x[r]
        best, other = int(l.argmax()), int(np.argsort(l)[-2])
        dvec = W[other] - W[best]
        x[r] += dvec * ((l[best] - l[other]) / float(dvec @ dvec))
        return dvec / float(dvec @ dvec), np.max(np.abs(l))

    ref_t, got_t = ref.copy(), ref.copy()
    for r in range(4):
        step, scale = make_tie(ref_t, r)
        eps = 1e-4 * scale                      # 10x inside TIE_REL
        ref_t[r] -= step * eps                  # the reference keeps `best` by eps
        got_t[r] = ref_t[r] + step * 2 * eps    # got tips to `other` by eps
    ref32, got32 = ref_t.astype(np.float32), got_t.astype(np.float32)
    rows, not_tie = argmax_mismatches(orc, got32, ref32, n)
    assert not not_tie
    # two flips in 200 rows are within the 1% cap ...
    one = ref32.copy()
    one[:2] = got32[:2]
    check(orc, one, ref32, 4, "bf16", n_queries=n, what="two ties")
    # ... four are not
    assert len(rows) == 4
    with pytest.raises(AssertionError, match="tie-flips"):
        check(orc, got32, ref32, 4, "bf16", n_queries=n, what="four ties")
