"""Pins the CPU oracle (oracle/attn_oracle.c) before anything is compared to it.

Each check is chosen so that a plausible restatement mistake (wrong GQA map,
off-by-one window, scale applied twice, wrong layer stride, dropped term)
fails at least one of them:
  * the reference's own known-answer tests, ported verbatim
    (forward.zig:297-364, math.zig:224-230 / 252-254, kv_cache.zig:198-282,
    pool.zig:196-259);
  * closed forms (L=1, constant K, one-hot score, softmax shift invariance);
  * invariants (window perturbation, GQA groups, prefill row b == decode at
    pos b, position permutation, pooled == single-threaded);
  * an independent vectorised numpy f64 formula of softmax(q K^T / sqrt(d)) V.
"""
import numpy as np
import pytest

from tests.util import np_attention_f64, rel_err, fill_cache_random


# ---------------------------------------------------------------- math.zig
def test_softmax_sums_to_1(orc):
    # math.zig:224-230
    x = orc.softmax(np.array([0.5, 1.5, -0.5, 2.0], np.float32))
    assert abs(float(x.sum()) - 1.0) <= 1e-5


def test_softmax_matches_closed_form_and_shift_invariance(orc):
    x = np.array([0.5, 1.5, -0.5, 2.0, -3.0], np.float32)
    e = np.exp(x.astype(np.float64) - x.max())
    ref = e / e.sum()
    got = orc.softmax(x)
    assert np.max(np.abs(got - ref)) < 1e-7
    got_shift = orc.softmax(x + np.float32(37.0))
    assert np.max(np.abs(got_shift - got)) < 1e-7
    assert orc.softmax(np.zeros(0, np.float32)).size == 0


def test_argmax(orc):
    # math.zig:252-254, plus first-max-wins (math.zig:190-201 uses '>')
    assert orc.argmax(np.array([0.1, 0.5, 1.5, 0.3], np.float32)) == 2
    assert orc.argmax(np.array([2.0, 1.0, 2.0], np.float32)) == 0
    assert orc.argmax(np.zeros(0, np.float32)) == 0


# ---------------------------------------------------------------- upcasts
def test_f16_upcast_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_upcast_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32)
    got = orc.bf16_bits_to_f32(bits.astype(np.uint16))
    assert np.array_equal(got.view(np.uint32), bits << 16)


def test_bf16_round_to_nearest_even(orc):
    u = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x7F7FFFFF, 0xFF800000],
                 np.uint32)
    got = orc.f32_to_bf16_bits(u.view(np.float32))
    assert list(got) == [0x3F80, 0x3F82, 0x3F81, 0x3F80, 0x7F80, 0xFF80]
    nan = orc.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(orc.bf16_bits_to_f32(nan))[0]


# ---------------------------------------------------------------- kv_cache.zig
def test_kvcache_slot_advance_round_trip(orc):
    # kv_cache.zig:198-225
    cache = orc.OracleKvCache(2, 4, 8, 16)
    assert cache.pos == 0
    cache.key_slot(0)[:] = np.arange(32)
    cache.value_slot(0)[:] = np.arange(32) * 10.0
    cache.key_slot(1)[:] = np.arange(32) + 0.5
    cache.advance()
    cache.key_slot(0)[:] = np.arange(32) + 100.0
    cache.advance()
    assert cache.pos == 2
    populated = cache.keys_for(0, cache.pos)
    assert populated.size == 2 * 4 * 8
    assert abs(populated[0] - 0) < 1e-6
    assert abs(populated[4 * 8] - 100) < 1e-6
    assert abs(cache.keys_for(1, 1)[0] - 0.5) < 1e-6


def test_kvcache_shrink_preserves_live_data(orc):
    # kv_cache.zig:227-263
    cache = orc.OracleKvCache(2, 4, 8, 64)
    for t in range(10):
        base = np.arange(32, dtype=np.float32) + t * 1000
        cache.key_slot(0)[:] = base
        cache.value_slot(0)[:] = base + 0.5
        cache.key_slot(1)[:] = base + 10000.0
        cache.value_slot(1)[:] = base + 10000.5
        cache.advance()
    assert cache.pos == 10
    cache.shrink_to_fit(32)
    assert cache.max_seq == 32 and cache.pos == 10
    l0 = cache.keys_for(0, 10)
    assert abs(l0[0]) < 1e-6 and abs(l0[9 * 32] - 9000) < 1e-6
    l1 = cache.keys_for(1, 10)
    assert abs(l1[0] - 10000) < 1e-6 and abs(l1[9 * 32] - 19000) < 1e-6
    for t in range(10, 32):
        cache.key_slot(0)[:] = np.arange(32) + t * 1000
        cache.advance()
    assert cache.pos == 32
    with pytest.raises(IndexError):
        cache.advance()


def test_kvcache_shrink_refuses_to_drop_entries(orc):
    # kv_cache.zig:265-282
    cache = orc.OracleKvCache(1, 2, 4, 32)
    for _ in range(20):
        cache.key_slot(0)[:] = 0
        cache.advance()
    with pytest.raises(ValueError):
        cache.shrink_to_fit(10)
    cache.shrink_to_fit(64)
    assert cache.max_seq == 32


# ---------------------------------------------------------------- window
def test_window_start_cases(orc):
    W = 4096
    assert orc.window_start(0) == 0
    assert orc.window_start(10**9) == 0
    assert orc.window_start(4095, W) == 0
    assert orc.window_start(4096, W) == 1
    assert orc.window_start(16383, W) == 12288
    assert orc.window_start(5, 3) == 3


def test_sliding_window_known_answer(orc):
    # forward.zig:297-364: 1 head, head_dim 2, window 3, pos 5.
    c = orc.config(1, 1, 2, 8, sliding_window=3)
    cache = orc.OracleKvCache(1, 1, 2, 8)
    K = cache.layer_rows("k", 0)
    V = cache.layer_rows("v", 0)
    for t in range(6):
        big = t < 3
        K[t, 0] = [100.0 if big else 1.0, 0.0]
        V[t, 0] = [-999.0 if big else 1.0, 0.0]
    cache.pos = 5
    out = orc.cpu_attention(np.array([1.0, 0.0], np.float32), cache, c, 0)
    assert abs(out[0] - 1.0) <= 1e-3
    assert out[0] > -100.0


# ---------------------------------------------------------------- closed forms
def test_single_row_returns_v(orc):
    # L=1: softmax of one score is 1, so out_h = v_{kv_h}.
    c = orc.config(8, 2, 16, 4)
    cache = orc.OracleKvCache(1, 2, 16, 4)
    fill_cache_random(orc, cache, 1, seed=3)
    cache.pos = 0
    q = orc.normal(5, 8 * 16)
    out = orc.cpu_attention(q, cache, c, 0).reshape(8, 16)
    V = cache.layer_rows("v", 0)
    for h in range(8):
        assert np.array_equal(out[h], V[0, (h * 2) // 8])


def test_constant_keys_give_mean_of_values(orc):
    n, d = 37, 16
    c = orc.config(2, 1, d, 64)
    cache = orc.OracleKvCache(1, 1, d, 64)
    K = cache.layer_rows("k", 0)
    V = cache.layer_rows("v", 0)
    K[:n, 0] = orc.normal(1, d)
    V[:n, 0] = orc.normal(2, n * d).reshape(n, d)
    cache.pos = n - 1
    out = orc.cpu_attention(orc.normal(3, 2 * d), cache, c, 0).reshape(2, d)
    mean = V[:n, 0].astype(np.float64).mean(axis=0)
    for h in range(2):
        assert np.max(np.abs(out[h] - mean)) < 1e-5


def test_one_hot_score_selects_row(orc):
    n, d = 20, 8
    c = orc.config(1, 1, d, 32)
    cache = orc.OracleKvCache(1, 1, d, 32)
    K = cache.layer_rows("k", 0)
    V = cache.layer_rows("v", 0)
    V[:n, 0] = orc.normal(4, n * d).reshape(n, d)
    K[:n, 0] = 0.0
    K[13, 0, 0] = 1000.0
    cache.pos = n - 1
    q = np.zeros(d, np.float32)
    q[0] = 1.0
    out = orc.cpu_attention(q, cache, c, 0)
    assert np.max(np.abs(out - V[13, 0])) < 1e-6


# ---------------------------------------------------------------- formula
@pytest.mark.parametrize("n_heads,n_kv,d,pos,window,layer", [
    (32, 4, 64, 511, None, 0),     # C1 shape
    (8, 8, 32, 100, None, 1),      # MHA, second layer
    (12, 4, 16, 300, 128, 2),      # GQA 3:1 + window
    (6, 4, 16, 50, None, 0),       # uneven GQA map (h*n_kv)/n_heads
    (4, 1, 256, 200, None, 0),     # MQA, head_dim 256
])
def test_decode_matches_independent_f64_formula(orc, n_heads, n_kv, d, pos, window, layer):
    max_seq = pos + 8
    W = orc.NO_WINDOW if window is None else window
    c = orc.config(n_heads, n_kv, d, max_seq, W)
    cache = orc.OracleKvCache(3, n_kv, d, max_seq)
    fill_cache_random(orc, cache, pos + 1, seed=11 + layer)
    cache.pos = pos
    q = orc.normal(99, n_heads * d) / np.float32(np.sqrt(d))
    got = orc.cpu_attention(q, cache, c, layer)
    ref = np_attention_f64(q, cache.layer_rows("k", layer), cache.layer_rows("v", layer),
                           n_heads, n_kv, d, pos, window)
    assert rel_err(got, ref, n_heads) <= 1e-5
    twin = orc.attention_f64(q, cache, c, layer, pos)
    assert rel_err(twin, ref, n_heads) <= 1e-12


def test_formula_check_detects_planted_mistakes(orc):
    """The f64 check is discriminative: mistakes planted in a CPU copy of the
    formula (GQA map, window off-by-one, double scaling) all exceed 1e-5."""
    n_heads, n_kv, d, pos, W = 8, 2, 16, 40, 16
    c = orc.config(n_heads, n_kv, d, 64, W)
    cache = orc.OracleKvCache(1, n_kv, d, 64)
    fill_cache_random(orc, cache, pos + 1, seed=7)
    cache.pos = pos
    q = orc.normal(8, n_heads * d)
    got = orc.cpu_attention(q, cache, c, 0)
    K, V = cache.layer_rows("k", 0), cache.layer_rows("v", 0)
    assert rel_err(got, np_attention_f64(q, K, V, n_heads, n_kv, d, pos, W), n_heads) <= 1e-5
    bad = [
        np_attention_f64(q, K, V, n_heads, n_kv, d, pos, W, kv_map=lambda h: h % n_kv),
        np_attention_f64(q, K, V, n_heads, n_kv, d, pos, W + 1),
        np_attention_f64(q, K, V, n_heads, n_kv, d, pos, W, scale=1.0 / d),
        np_attention_f64(q, K, V, n_heads, n_kv, d, pos - 1, W),
    ]
    for b in bad:
        assert rel_err(got, b, n_heads) > 1e-3


# ---------------------------------------------------------------- invariants
def test_output_independent_of_rows_outside_window(orc):
    n_heads, n_kv, d, pos, W = 4, 2, 16, 90, 32
    c = orc.config(n_heads, n_kv, d, 128, W)
    cache = orc.OracleKvCache(1, n_kv, d, 128)
    fill_cache_random(orc, cache, pos + 1, seed=21)
    cache.pos = pos
    q = orc.normal(22, n_heads * d)
    a = orc.cpu_attention(q, cache, c, 0)
    ws = orc.window_start(pos, W)
    cache.layer_rows("k", 0)[:ws] = 1e4
    cache.layer_rows("v", 0)[:ws] = -1e4
    cache.layer_rows("k", 0)[pos + 1:] = 1e4  # rows after pos are never read either
    b = orc.cpu_attention(q, cache, c, 0)
    assert np.array_equal(a, b)
    cache.layer_rows("v", 0)[ws] += 1.0  # first in-window row does matter
    assert not np.array_equal(a, orc.cpu_attention(q, cache, c, 0))


def test_gqa_group_members_with_equal_q_agree(orc):
    n_heads, n_kv, d, pos = 8, 2, 16, 30
    c = orc.config(n_heads, n_kv, d, 64)
    cache = orc.OracleKvCache(1, n_kv, d, 64)
    fill_cache_random(orc, cache, pos + 1, seed=31)
    cache.pos = pos
    qh = orc.normal(32, d)
    q = np.tile(qh, n_heads)
    out = orc.cpu_attention(q, cache, c, 0).reshape(n_heads, d)
    for h in range(1, 4):
        assert np.array_equal(out[h], out[0])
    assert not np.array_equal(out[4], out[0])


def test_prefill_row_equals_decode_at_that_position(orc):
    # prefill.zig:21-23: byte-equal to B single-token steps.
    n_heads, n_kv, d, B, pos0, W = 4, 2, 16, 24, 5, 8
    for window in (orc.NO_WINDOW, W):
        c = orc.config(n_heads, n_kv, d, 64, window)
        cache = orc.OracleKvCache(1, n_kv, d, 64)
        fill_cache_random(orc, cache, pos0 + B, seed=41)
        q_all = orc.normal(42, B * n_heads * d)
        cache.pos = pos0
        rows = list(range(B))
        pre = orc.attention_causal(q_all, cache, c, 0, rows)
        for b in rows:
            cache.pos = pos0 + b
            dec = orc.cpu_attention(q_all[b * n_heads * d:(b + 1) * n_heads * d], cache, c, 0)
            assert np.array_equal(pre[b], dec)
        cache.pos = pos0


def test_position_permutation_invariance(orc):
    n_heads, n_kv, d, pos = 4, 4, 16, 63
    c = orc.config(n_heads, n_kv, d, 64)
    cache = orc.OracleKvCache(1, n_kv, d, 64)
    fill_cache_random(orc, cache, pos + 1, seed=51)
    cache.pos = pos
    q = orc.normal(52, n_heads * d)
    a = orc.cpu_attention(q, cache, c, 0)
    perm = np.random.default_rng(0).permutation(pos + 1)
    for which in ("k", "v"):
        rows = cache.layer_rows(which, 0)
        rows[:pos + 1] = rows[:pos + 1][perm]
    b = orc.cpu_attention(q, cache, c, 0)
    assert rel_err(a, b, n_heads) <= 1e-6


# ---------------------------------------------------------------- pool.zig
def test_pool_sums_chunks(orc):
    # pool.zig:196-221
    pool = orc.Pool(4)
    try:
        data = np.arange(1, 1001, dtype=np.uint32)
        assert pool.sum(data) == 500500
        pool.set_active(2)
        assert pool.sum(data) == 500500
        pool.set_active(100)  # clamped to n_workers (pool.zig:127-130)
        assert pool.sum(data) == 500500
    finally:
        pool.close()


def test_pooled_attention_bit_identical(orc):
    n_heads, n_kv, d, pos = 32, 4, 64, 511
    c = orc.config(n_heads, n_kv, d, 512)
    cache = orc.OracleKvCache(1, n_kv, d, 512)
    fill_cache_random(orc, cache, pos + 1, seed=61)
    cache.pos = pos
    q = orc.normal(62, n_heads * d)
    pool = orc.Pool(4)
    try:
        assert np.array_equal(pool.attention(q, cache, c, 0, pos), orc.cpu_attention(q, cache, c, 0))
    finally:
        pool.close()


# ---------------------------------------------------------------- RNG
def test_rng_is_counter_based_and_normal(orc):
    a = orc.normal(0, 1000)
    b = orc.normal(0, 500, offset=500)
    assert np.array_equal(a[500:], b)
    assert not np.array_equal(orc.normal(1, 10), a[:10])
    big = orc.normal(123, 200000).astype(np.float64)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01
    # Pinned first values (regression guard for the committed golden vectors).
    assert orc.splitmix64(0, np.array([0], np.uint64))[0] == np.uint64(0xE220A8397B1DCDAF)
