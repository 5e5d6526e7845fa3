"""The prefill kernel's precision choice (prefill_entry in
vantablack_amd/csrc/kernels/prefill.hip), checked on the CPU:

  - q rounded to f16 after the kernel's power-of-two scale moves each
    element by at most 2^-11 of itself (f16's unit roundoff), so a score
    q.k moves by at most 2^-11 * sum |q_i k_i| <= 2^-11 * |q| |k|: in log2
    units 2^-11 * B, B = |q| |k| * scale_log2, which is 2^-6 at the
    threshold B = 32.  The bound holds on random data and is reached (to
    within a few percent) by a constructed worst case, so 2^-6 is the right
    figure, not a loose one.
  - bench.prefill_paths, which reports the share of work items taking each
    form, applies the kernel's rule: two-piece q iff max|q| * max|k_t| *
    scale_log2 > 32 over the item's key tiles, two-piece P iff the values'
    crest factor over those tiles exceeds 8.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LOG2E = 1.4426950408889634


def f16_round_scaled(x):
    """The kernel's q conversion: scale by 2^-e (largest |x| into
    [2^14, 2^15)), round to f16, scale back (exact)."""
    m = np.abs(x).max()
    e = int(np.floor(np.log2(m))) - 14
    return (x * 2.0 ** -e).astype(np.float16).astype(np.float64) * 2.0 ** e


@pytest.mark.parametrize("d", [64, 128, 256])
def test_score_error_within_the_bound(d):
    rng = np.random.default_rng(d)
    for scale in (1.0, 40.0, 1e-3):
        q = rng.standard_normal((64, d)) * scale
        k = rng.standard_normal((64, d))
        qr = np.stack([f16_round_scaled(row) for row in q])
        err = np.abs((qr - q) @ k.T)                          # |score error|
        bound = 2.0 ** -11 * np.abs(q) @ np.abs(k).T           # 2^-11 sum |q_i k_i|
        cs = 2.0 ** -11 * np.outer(np.linalg.norm(q, axis=1), np.linalg.norm(k, axis=1))
        assert (err <= bound * (1 + 1e-12)).all()
        assert (bound <= cs * (1 + 1e-12)).all()


def test_bound_is_reached_by_a_worst_case():
    # q_i just above 1 + 2^-11 (rounds down to 1 in f16: error ~2^-11 of
    # q_i, all of one sign) and k_i = 1: the error is ~2^-11 |q| |k|.
    d = 128
    q = np.full(d, 1.0 + 2.0 ** -11 * (1 - 2.0 ** -12))
    q[0] = 1.5  # sets the scale: max in [2^14, 2^15) after 2^-e
    k = np.ones(d)
    err = abs((f16_round_scaled(q) - q) @ k)
    cs = 2.0 ** -11 * np.linalg.norm(q) * np.linalg.norm(k)
    assert err > 0.95 * cs
    # At the selection threshold B = |q||k| scale_log2 = 32 this is 2^-6
    # in log2 units: exp2 of it moves P by about 1.1%.
    assert abs(2.0 ** -11 * 32 - 2.0 ** -6) < 1e-15
    assert 0.010 < 2.0 ** (2.0 ** -6) - 1 < 0.011


def test_kernel_rule_constants():
    src = open(os.path.join(ROOT, "vantablack_amd", "csrc", "kernels", "prefill.hip")).read()
    assert "const bool xq = sqrtf(qn2) * sqrtf(kn2) * a.scale_log2 > 32.0f;" in src
    assert "const bool xp = (double)vmx * vmx * ((double)cnt * D) > 64.0 * (double)vss;" in src
    assert "32: f16 rounding moves each q element by at most 2^-11 of itself, so" in src
    assert "a score by at most 2^-11 * B, which is 2^-6 at the threshold." in src


def _paths(q, k, v, inv):
    torch = pytest.importorskip("torch")
    sys.path.insert(0, ROOT)
    import bench
    return bench.prefill_paths(torch, torch.tensor(q, dtype=torch.float32), torch.tensor(k, dtype=torch.float32),
                               torch.tensor(v, dtype=torch.float32), inv)


def test_reported_paths_follow_the_rule():
    d, B, nh, nkv = 64, 256, 2, 1   # two blocks of 128 queries per head
    inv = 1.0 / np.sqrt(d)
    unit = np.zeros(d)
    unit[0] = 1.0
    # Every q row of norm a, every k row of norm b: B = a b scale_log2.
    for a, b in ((10.0, 15.0), (10.0, 20.0)):  # B = 27.0 and 36.1
        q = np.tile(unit * a, (B, nh, 1))
        k = np.tile(unit * b, (B, nkv, 1))
        v = np.ones((B, nkv, d))
        p = _paths(q, k, v, inv)
        want = a * b * inv * LOG2E > 32.0
        assert p["xq_frac"] == (1.0 if want else 0.0), (a, b, p)
        assert p["xp_frac"] == 0.0  # constant values: crest 1
    # Values: one row at 100 among rows of 1 in the first block's keys (crest
    # ~11 over either block's range, which both include that row), then at
    # 1.5 (crest ~1.5).
    q = np.tile(unit, (B, nh, 1))
    k = np.tile(unit, (B, nkv, 1))
    v = np.ones((B, nkv, d))
    v[3, 0, :] = 100.0
    p = _paths(q, k, v, inv)
    assert p["xp_frac"] == 1.0 and p["xq_frac"] == 0.0
    v[3, 0, :] = 1.5
    assert _paths(q, k, v, inv)["xp_frac"] == 0.0
