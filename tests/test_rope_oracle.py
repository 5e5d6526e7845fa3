"""Pins the oracle's RoPE (math.rope / math.ropeHalf, src/kernels/math.zig:85-133)
before the fused decode prologue is compared to it.

A plausible restatement mistake -- pairing i with i+1 in the half form,
indexing the frequency by i instead of 2i, a sign flip in the rotation, the
exponent computed as an integer quotient -- fails at least one of:
  * the reference's known-answer test (math.zig:217-222);
  * pair 0 (inv_freq exactly 1) is the textbook rotation by pos radians;
  * the frequency table against 1 / base^(2j/d) in f64;
  * the rotation against an independent f64 formula;
  * ropeHalf equals rope under the half <-> interleaved permutation, bit for bit;
  * pair norms are preserved and rotations by a and b compose to a + b.
"""
import numpy as np
import pytest


def _interleave(x):
    """Half layout (x[j], x[j+d/2]) -> interleaved (y[2j], y[2j+1])."""
    d = x.shape[-1]
    y = np.empty_like(x)
    y[..., 0::2] = x[..., : d // 2]
    y[..., 1::2] = x[..., d // 2:]
    return y


def _deinterleave(y):
    d = y.shape[-1]
    x = np.empty_like(y)
    x[..., : d // 2] = y[..., 0::2]
    x[..., d // 2:] = y[..., 1::2]
    return x


def _f64_rope(x, pos, base, half):
    """Independent formula: rotation of each pair by pos * base^(-2j/d)."""
    x = x.astype(np.float64)
    d = x.shape[-1]
    j = np.arange(d // 2, dtype=np.float64)
    theta = pos * base ** (-2.0 * j / d)
    c, s = np.cos(theta), np.sin(theta)
    if half:
        a, b = x[..., : d // 2], x[..., d // 2:]
    else:
        a, b = x[..., 0::2], x[..., 1::2]
    ra, rb = a * c - b * s, a * s + b * c
    out = np.empty_like(x)
    if half:
        out[..., : d // 2], out[..., d // 2:] = ra, rb
    else:
        out[..., 0::2], out[..., 1::2] = ra, rb
    return out


def test_rope_zero_position_is_identity(orc):
    # math.zig:217-222
    x = orc.rope(np.array([1.0, 2.0, 3.0, 4.0], np.float32), 0, 10000.0)
    assert abs(float(x[0]) - 1.0) <= 1e-5 and abs(float(x[1]) - 2.0) <= 1e-5
    # cos 0 = 1 and sin 0 = 0 exactly: both forms are the identity at pos 0.
    v = orc.normal(3, 256).reshape(2, 128)
    assert np.array_equal(orc.rope(v, 0, 10000.0), v)
    assert np.array_equal(orc.rope(v, 0, 10000.0, half=True), v)


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("pos", [1, 7, 1000, 4095])
def test_rope_first_pair_is_rotation_by_pos(orc, pos, half):
    d = 64
    x = orc.normal(11, d)
    y = orc.rope(x, pos, 10000.0, half=half)
    i0, i1 = (0, d // 2) if half else (0, 1)
    c, s = np.cos(float(pos)), np.sin(float(pos))
    x0, x1 = float(x[i0]), float(x[i1])
    assert abs(float(y[i0]) - (x0 * c - x1 * s)) <= 2e-6 * (abs(x0) + abs(x1))
    assert abs(float(y[i1]) - (x0 * s + x1 * c)) <= 2e-6 * (abs(x0) + abs(x1))


@pytest.mark.parametrize("d,base", [(64, 10000.0), (128, 500000.0), (256, 1000000.0)])
def test_rope_inv_freq_table(orc, d, base):
    t = orc.rope_inv_freq(d, base).astype(np.float64)
    ref = base ** (-2.0 * np.arange(d // 2) / d)
    assert t[0] == 1.0
    assert np.max(np.abs(t - ref) / ref) <= 3e-7


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("pos", [1, 17, 1000, 30000])
def test_rope_matches_f64_formula(orc, d, pos, half):
    base = 10000.0
    x = orc.normal(100 + d + pos, 8 * d).reshape(8, d)
    y = orc.rope(x, pos, base, half=half).astype(np.float64)
    ref = _f64_rope(x, pos, base, half)
    # The f32 angle pos * inv_freq carries ~pos * 2^-24 of absolute error.
    tol = 4e-6 + 2.0 * pos * 2.0 ** -24
    assert np.max(np.abs(y - ref)) <= tol * np.max(np.abs(x))


def test_rope_f64_check_detects_planted_mistakes(orc):
    """The f64 comparison above fails for the likely wrong variants."""
    d, pos, base = 128, 1000, 10000.0
    x = orc.normal(5, d)
    ref = _f64_rope(x, pos, base, half=False)
    good = orc.rope(x, pos, base).astype(np.float64)
    tol = 4e-6 + 2.0 * pos * 2.0 ** -24
    assert np.max(np.abs(good - ref)) <= tol * np.max(np.abs(x))
    # half-form pairing applied where interleaved was meant
    wrong_pair = orc.rope(x, pos, base, half=True).astype(np.float64)
    # frequency indexed by i instead of 2i (a different base schedule)
    wrong_freq = _f64_rope(x, pos, base ** 2, half=False)
    # rotation sign flipped (rotation by -theta)
    wrong_sign = _f64_rope(x, -pos, base, half=False)
    for bad in (wrong_pair, wrong_freq, wrong_sign):
        assert np.max(np.abs(bad - ref)) > 100 * tol * np.max(np.abs(x))


@pytest.mark.parametrize("pos", [3, 999, 30000])
def test_rope_half_is_permuted_rope(orc, pos):
    x = orc.normal(21, 4 * 128).reshape(4, 128)
    a = orc.rope(x, pos, 10000.0, half=True)
    b = _deinterleave(orc.rope(_interleave(x), pos, 10000.0))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("half", [False, True])
def test_rope_preserves_pair_norms_and_composes(orc, half):
    d, base = 128, 10000.0
    x = orc.normal(31, d)
    y = orc.rope(x, 123, base, half=half).astype(np.float64)
    xx = x.astype(np.float64)
    if half:
        n0 = xx[: d // 2] ** 2 + xx[d // 2:] ** 2
        n1 = y[: d // 2] ** 2 + y[d // 2:] ** 2
    else:
        n0 = xx[0::2] ** 2 + xx[1::2] ** 2
        n1 = y[0::2] ** 2 + y[1::2] ** 2
    assert np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-12)) <= 2e-6
    two = orc.rope(orc.rope(x, 40, base, half=half), 60, base, half=half).astype(np.float64)
    one = orc.rope(x, 100, base, half=half).astype(np.float64)
    assert np.max(np.abs(two - one)) <= 2e-5 * np.max(np.abs(xx))
