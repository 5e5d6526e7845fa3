"""Pins the oracle's batched matmul (vtb_oracle_matmul_batched, restating
src/runtime/prefill.zig:325-378 matmulBatched: dequantToF32 of a whole row,
then simd.dot_f32 with every token, simd.zig:13-29) before the GPU kernel is
compared to it:
  * bit-equality with an independent numpy restatement of dot_f32's order
    (eight lane accumulators over the row, products rounded before the add,
    lane-order reduction) on the independently dequantised weights;
  * the f64 dot, within 1e-6 of sum |W||x| per output;
  * a batch of identical tokens gives identical rows;
  * a planted order mistake (per-block reduction, as the single-token
    matmul_* do) is caught by the bit-equality check.
"""
import numpy as np
import pytest

from tests.quant import BLOCK, np_dequant, random_weights

KINDS = ["q8_0", "q4_k", "q5_k", "q6_k"]


def np_dot_f32(W, X):
    """out[t, r] per simd.dot_f32: acc[l] += W[r, i+l] * X[t, i+l] over i in
    steps of 8 (f32, product rounded first), then ((acc0 + acc1) + acc2) ...
    """
    m, k = W.shape
    B = X.shape[0]
    Wv = W.reshape(m, k // 8, 8).astype(np.float32)
    Xv = X.reshape(B, k // 8, 8).astype(np.float32)
    acc = np.zeros((B, m, 8), np.float32)
    for i in range(k // 8):
        prod = (Xv[:, None, i, :] * Wv[None, :, i, :]).astype(np.float32)
        acc = (acc + prod).astype(np.float32)
    s = acc[:, :, 0].copy()
    for l in range(1, 8):
        s = (s + acc[:, :, l]).astype(np.float32)
    return s


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m,k,B", [(5, 512, 3), (3, 1024, 7)])
def test_matches_independent_numpy_bit_for_bit(orc, kind, m, k, B):
    w = random_weights(kind, m, k, seed=m * 31 + k + B)
    x = orc.normal(k + B, B * k).reshape(B, k)
    got = orc.matmul_batched(kind, w, x, m, k, B)
    ref = np_dot_f32(np_dequant(kind, w).reshape(m, k), x)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("kind", KINDS)
def test_matches_f64_dot(orc, kind):
    m, k, B = 6, 2048, 4
    w = random_weights(kind, m, k, seed=17)
    x = orc.normal(18, B * k).reshape(B, k)
    got = orc.matmul_batched(kind, w, x, m, k, B).astype(np.float64)
    W = np_dequant(kind, w).astype(np.float64).reshape(m, k)
    ref = x.astype(np.float64) @ W.T
    cond = np.abs(x.astype(np.float64)) @ np.abs(W).T
    assert np.all(np.abs(got - ref) <= 1e-6 * cond)


def test_identical_tokens_give_identical_rows(orc):
    m, k, B = 4, 512, 5
    w = random_weights("q4_k", m, k, seed=3)
    x = np.tile(orc.normal(4, k), (B, 1))
    got = orc.matmul_batched("q4_k", w, x, m, k, B)
    assert all(np.array_equal(got[0], got[b]) for b in range(B))


def test_order_mistake_is_caught(orc):
    # the single-token matmul_q4_k reduces per block; matmulBatched does not
    m, k = 8, 4096
    w = random_weights("q4_k", m, k, seed=21)
    x = orc.normal(22, k)
    batched = orc.matmul_batched("q4_k", w, x.reshape(1, k), m, k, 1)[0]
    per_block = orc.matmul_quant("q4_k", w, x, m, k)
    assert not np.array_equal(batched, per_block)
    assert np.array_equal(batched, np_dot_f32(np_dequant("q4_k", w).reshape(m, k), x.reshape(1, k))[0])


def test_rejects_k_above_max(orc):
    with pytest.raises(ValueError):
        orc.matmul_batched("q8_0", np.zeros(34 * 1025, np.uint8), np.zeros(32800, np.float32), 1, 32800, 1)
