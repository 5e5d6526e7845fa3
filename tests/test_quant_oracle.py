"""Pins the oracle's quantised matmuls (oracle/quant_oracle.c, restating
src/kernels/simd.zig) before the GPU GEMV is compared to them:
  * the reference's own known-answer tests, ported (simd.zig:586-720);
  * an independent vectorised numpy dequantiser (tests/quant.py), which must
    agree bit for bit on random blocks -- with planted layout mistakes
    (scale/min unpacking, Q5_K fifth bit, Q6_K bias) shown to break it;
  * the matmul against an f64 dot of the dequantised weights.
"""
import numpy as np
import pytest

from tests.quant import BLOCK, np_dequant, random_weights

KINDS = ["q8_0", "q4_k", "q5_k", "q6_k"]


def _f16bits(v):
    return int(np.float16(v).view(np.uint16))


def test_q8_0_dequant_round_trips(orc):
    # simd.zig:586-599
    block = np.zeros(34, np.uint8)
    block[0:2] = np.array([_f16bits(0.125)], np.uint16).view(np.uint8)
    qs = np.array([-64, -32, -16, -8, -4, -2, -1, 0, 1, 2, 4, 8, 16, 32, 64, 100, -100, 50, -50, 25, -25, 12,
                   -12, 6, -6, 3, -3, 1, -1, 0, 0, 0], np.int8)
    block[2:] = qs.view(np.uint8)
    out = orc.dequant("q8_0", block)
    assert np.max(np.abs(out - 0.125 * qs.astype(np.float32))) <= 1e-4


def _q4k_block():
    # simd.zig:601-626
    block = np.zeros(144, np.uint8)
    block[0:2] = np.array([_f16bits(0.0078125)], np.uint16).view(np.uint8)
    block[2:4] = np.array([_f16bits(0.0625)], np.uint16).view(np.uint8)
    for s in range(4):
        block[4 + s] = (s + 1) * 5
        block[8 + s] = s + 2
    for s in range(4):
        block[12 + s] = ((s + 1) * 3) | ((s + 1) << 4)
    for i in range(128):
        block[16 + i] = ((i * 7) % 16) | (((i * 11) % 16) << 4)
    return block


def test_q4_k_dequant_and_matmul_self_consistent(orc):
    # simd.zig:601-651
    block = _q4k_block()
    dq = orc.dequant("q4_k", block)
    d, dmin = np.float32(0.0078125), np.float32(0.0625)
    exp0 = d * np.float32(block[4] & 0x3F) * np.float32(block[16] & 0x0F) - dmin * np.float32(block[8] & 0x3F)
    assert abs(dq[0] - exp0) <= 1e-4
    exp_sb1 = d * np.float32(block[5] & 0x3F) * np.float32(block[16] >> 4) - dmin * np.float32(block[9] & 0x3F)
    assert abs(dq[32] - exp_sb1) <= 1e-4
    x = (np.arange(256) % 7).astype(np.float32) * np.float32(0.1)
    got = orc.matmul_quant("q4_k", block, x, 1, 256)
    assert abs(float(got[0]) - float(np.dot(dq.astype(np.float64), x))) <= 1e-3


def test_q5_k_dequant_and_matmul_self_consistent(orc):
    # simd.zig:653-697
    block = np.zeros(176, np.uint8)
    block[0:2] = np.array([_f16bits(0.00390625)], np.uint16).view(np.uint8)
    block[2:4] = np.array([_f16bits(0.03125)], np.uint16).view(np.uint8)
    for s in range(4):
        block[4 + s] = (s + 1) * 4
        block[8 + s] = s + 1
        block[12 + s] = ((s + 1) * 2) | ((s + 1) << 4)
    for l in range(32):
        block[16 + l] = (l * 31) % 256
    for i in range(128):
        block[48 + i] = ((i * 13) % 16) | (((i * 7) % 16) << 4)
    dq = orc.dequant("q5_k", block)
    w5_0 = (block[48] & 0x0F) + (16 if block[16] & 1 else 0)
    exp0 = np.float32(0.00390625) * np.float32(block[4] & 0x3F) * np.float32(w5_0) - \
        np.float32(0.03125) * np.float32(block[8] & 0x3F)
    assert abs(dq[0] - exp0) <= 1e-4
    x = (np.arange(256) % 9).astype(np.float32) * np.float32(0.1) - np.float32(0.4)
    got = orc.matmul_quant("q5_k", block, x, 1, 256)
    assert abs(float(got[0]) - float(np.dot(dq.astype(np.float64), x))) <= 1e-3


def test_q6_k_dequant_and_matmul_self_consistent(orc):
    # simd.zig:699-733
    block = np.zeros(210, np.uint8)
    block[208:210] = np.array([_f16bits(0.001953125)], np.uint16).view(np.uint8)
    for i in range(128):
        block[i] = (i * 17) % 256
    for i in range(64):
        block[128 + i] = (i * 19) % 256
    block[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    dq = orc.dequant("q6_k", block)
    q1 = int((block[0] & 0x0F) | ((block[128] & 3) << 4)) - 32
    exp0 = np.float32(0.001953125) * np.float32(np.int8(block[192].view(np.int8))) * np.float32(q1)
    assert abs(dq[0] - exp0) <= 1e-4
    x = (np.arange(256) % 11).astype(np.float32) * np.float32(0.05) - np.float32(0.25)
    got = orc.matmul_quant("q6_k", block, x, 1, 256)
    assert abs(float(got[0]) - float(np.dot(dq.astype(np.float64), x))) <= 1e-3


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_matches_independent_numpy(orc, kind):
    w = random_weights(kind, 8, 1024, seed=11)
    assert np.array_equal(orc.dequant(kind, w), np_dequant(kind, w))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m,k", [(4, 512), (16, 4096), (3, 8192)])
def test_matmul_matches_f64_dot(orc, kind, m, k):
    if k % BLOCK[kind][1]:
        pytest.skip("not a whole number of blocks")
    w = random_weights(kind, m, k, seed=m + k)
    x = orc.normal(m * 7 + k, k)
    got = orc.matmul_quant(kind, w, x, m, k).astype(np.float64)
    W = np_dequant(kind, w).astype(np.float64).reshape(m, k)
    ref = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))     # condition of each row's sum
    assert np.all(np.abs(got - ref) <= 1e-6 * scale)


def test_independent_dequant_detects_planted_mistakes(orc):
    """The numpy/C agreement would break for the likely layout mistakes."""
    import tests.quant as tq
    w = random_weights("q4_k", 4, 1024, seed=5)
    good = orc.dequant("q4_k", w)
    b = w.reshape(-1, 144).copy()
    # 1. sub-blocks 4..7 taking the high bits from the wrong byte
    wrong = b.copy()
    wrong[:, 4:8], wrong[:, 8:12] = b[:, 8:12], b[:, 4:8]
    assert not np.array_equal(tq.np_dequant("q4_k", wrong), good)
    # 2. Q5_K without the fifth bit equals Q4_K of the same nibbles
    w5 = random_weights("q5_k", 2, 512, seed=6).reshape(-1, 176)
    as4 = np.concatenate([w5[:, :16], w5[:, 48:]], axis=1)
    assert not np.array_equal(orc.dequant("q5_k", w5), orc.dequant("q4_k", as4))
    # 3. Q6_K bias: with every ql/qh bit clear each weight is d * sc * (-32)
    #    exactly, sc taken per 16 weights in the reference's order
    w6 = random_weights("q6_k", 1, 256, seed=7).reshape(210).copy()
    w6[0:192] = 0
    d = np.float32(w6[208:210].copy().view(np.float16)[0])
    sc = w6[192:208].view(np.int8).astype(np.float32)
    idx = np.array([(p // 128) * 8 + (p % 128 % 32) // 16 + 2 * ((p % 128) // 32) for p in range(256)])
    assert np.array_equal(orc.dequant("q6_k", w6), (d * sc[idx]) * np.float32(-32))
