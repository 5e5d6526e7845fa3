"""kv_cache.zig's own tests (:198-282) run against the device-resident
KvCache, plus the f32 -> f16/bf16 slot-append rounding, bit-exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _write_slot(ctx, cache, layer, which, values):
    import vantablack_amd as vb
    src = ctx.to_device(np.asarray(values, np.float32))
    buf = cache.k if which == "k" else cache.v
    with ctx.segment() as seg:
        seg.kv_append(buf, cache.slot_offset(layer), cache.dtype, src, 0, cache.row_elems)
    ctx.wait_idle()


def test_kvcache_slot_advance_round_trip(ctx):
    import vantablack_amd as vb
    cache = vb.KvCache(ctx, 2, 4, 8, 16, "f32")
    try:
        assert cache.pos == 0
        _write_slot(ctx, cache, 0, "k", np.arange(32))
        _write_slot(ctx, cache, 0, "v", np.arange(32) * 10.0)
        _write_slot(ctx, cache, 1, "k", np.arange(32) + 0.5)
        cache.advance()
        _write_slot(ctx, cache, 0, "k", np.arange(32) + 100.0)
        cache.advance()
        assert cache.pos == 2
        populated = cache.read_rows("k", 0, cache.pos).reshape(-1)
        assert populated.size == 2 * 4 * 8
        assert abs(populated[0]) < 1e-6 and abs(populated[4 * 8] - 100) < 1e-6
        assert abs(cache.read_rows("k", 1, 1).reshape(-1)[0] - 0.5) < 1e-6
    finally:
        cache.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_kvcache_shrink_preserves_live_data(ctx, orc, dtype):
    import vantablack_amd as vb
    cache = vb.KvCache(ctx, 2, 4, 8, 64, dtype)
    try:
        for t in range(10):
            base = np.arange(32, dtype=np.float32) + t * 1000
            _write_slot(ctx, cache, 0, "k", base)
            _write_slot(ctx, cache, 0, "v", base + 0.5)
            _write_slot(ctx, cache, 1, "k", base + 10000.0)
            _write_slot(ctx, cache, 1, "v", base + 10000.5)
            cache.advance()
        cache.shrink_to_fit(32)
        assert cache.max_seq == 32 and cache.pos == 10

        def rd(which, layer):
            r = cache.read_rows(which, layer, 10).reshape(-1)
            return r if dtype == "f32" else (r.astype(np.uint32) << 16).view(np.float32)

        def stored(x):  # the value the cache holds after rounding to its dtype
            x = np.float32(x)
            return x if dtype == "f32" else orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.array([x])))[0]
        l0, l1 = rd("k", 0), rd("k", 1)
        assert l0[0] == 0 and l0[9 * 32] == stored(9000)
        assert l1[0] == stored(10000) and l1[9 * 32] == stored(19000)
        # every live row of both layers survives compaction exactly
        for layer, off in ((0, 0.0), (1, 10000.0)):
            want = np.concatenate([np.arange(32, dtype=np.float32) + t * 1000 + off for t in range(10)])
            want = want if dtype == "f32" else orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(want))
            assert np.array_equal(rd("k", layer), want)
        for t in range(10, 32):
            _write_slot(ctx, cache, 0, "k", np.arange(32) + t * 1000)
            cache.advance()
        assert cache.pos == 32
        with pytest.raises(vb.KvCacheFull):
            cache.advance()
    finally:
        cache.close()


def test_kvcache_shrink_refuses_to_drop_entries(ctx):
    import vantablack_amd as vb
    cache = vb.KvCache(ctx, 1, 2, 4, 32, "f16")
    try:
        cache.pos = 20
        with pytest.raises(vb.NewMaxSeqBelowPos):
            cache.shrink_to_fit(10)
        cache.shrink_to_fit(64)
        assert cache.max_seq == 32
    finally:
        cache.close()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_kv_append_rounds_to_nearest_even(ctx, orc, dtype):
    import vantablack_amd as vb
    rng = np.random.default_rng(1)
    x = np.concatenate([
        orc.normal(3, 4096) * np.float32(3.0),
        rng.standard_normal(1024).astype(np.float32) * np.float32(1e-6),  # f16 subnormals
        np.array([65504.0, 65520.0, 1e6, -1e6, 0.0, -0.0, np.inf, -np.inf], np.float32),
        (np.array([0x3F808000, 0x3F818000, 0x3F80FFFF], np.uint32)).view(np.float32),
    ]).astype(np.float32)
    n = x.size + 3  # odd length exercises the scalar tail
    x = np.concatenate([x, np.float32([1.5, -2.25, 3.0])])
    want = orc.f32_to_f16_bits(x) if dtype == "f16" else orc.f32_to_bf16_bits(x)
    src = ctx.to_device(x)
    dst = ctx.alloc(n * 2 + 16)
    for off in (0, 2):  # aligned (vector) and unaligned (scalar) destinations
        with ctx.segment() as seg:
            seg.kv_append(dst, off, vb.hip.DTYPES[dtype], src, 0, n)
        got = ctx.download(dst, np.uint16, n, offset=off)
        assert np.array_equal(got, want)


def test_segment_copy(ctx):
    x = np.arange(1000, dtype=np.float32)
    src = ctx.to_device(x)
    dst = ctx.to_device(np.zeros(1100, np.float32))
    with ctx.segment() as seg:
        seg.copy(dst, 40, src, 8, 900)
    got = ctx.download(dst, np.float32, 1100)
    assert np.array_equal(got[10:910], x[2:902]) and np.all(got[:10] == 0) and np.all(got[910:] == 0)
