"""The decode configs at their exact points, through the C ABI.

C2 (Llama-2-7B shapes) as BASELINE.json writes it: 32 layers x 32/32 heads x
d128, f16 KV already holding 4096 rows, decoded token after token through
the host mirror of stepWithBackend (forward.zig:152-172): one layer_step per
layer (KV-slot write + decode attention in one launch), one cache.advance()
per token (kv_cache.zig:130-133), finalize_token.  Every (layer, step) output
is checked against forward.cpuAttention restated (oracle.cpu_attention, split
over heads on the oracle's pool.zig-style pool) and every step's appended
K/V row bit-exactly against f32 -> f16 round to nearest even.  Two runs:
every step of a reduced stretch (L = 4097 .. 4096 + STEPS), and all 256
steps of the config (L = 4097 .. 4352) with the outputs of steps 0, 1, 127
and 255 checked on every layer and every appended row checked at the end.

C5 decode (Gemma shapes) at L = 32768: 8 q heads, 1 KV head, d256, bf16,
the layer-level entry on layer 1 of a two-layer cache.
"""
import numpy as np
import pytest

from tests.parity import check, decode_case

pytestmark = pytest.mark.gpu

C2_LAYERS, C2_HEADS, C2_D, C2_L0, C2_STEPS = 32, 32, 128, 4096, 6


_BASE = {}


def _layer_kv(layer):
    """Layer l's rows [0, C2_L0) of K and V as f16: rows [l, l + C2_L0) of
    one seeded N(0,1) base array per tensor, so every layer's prefix differs
    (a wrong layer offset reads different values) while only two arrays are
    ever drawn."""
    if not _BASE:
        rng = np.random.default_rng(1000)
        for which in ("k", "v"):
            _BASE[which] = rng.standard_normal((C2_L0 + C2_LAYERS, C2_HEADS, C2_D), dtype=np.float32).astype(
                np.float16)
    return _BASE["k"][layer:layer + C2_L0], _BASE["v"][layer:layer + C2_L0]


def _step_inputs(layer, step):
    """q ~ N(0,1)/sqrt(128) and the token's k_cur / v_cur ~ N(0,1), f32."""
    rng = np.random.default_rng(50000 + 100 * layer + step)
    q = (rng.standard_normal(C2_HEADS * C2_D, dtype=np.float32) / np.float32(np.sqrt(C2_D))).astype(np.float32)
    kc = rng.standard_normal(C2_HEADS * C2_D, dtype=np.float32)
    vc = rng.standard_normal(C2_HEADS * C2_D, dtype=np.float32)
    return q, kc, vc


def test_c2_step_sequence_through_the_backend(ctx, orc):
    import vantablack_amd as vb
    max_seq = C2_L0 + C2_STEPS
    c = vb.LlamaConfig(C2_HEADS, C2_HEADS, C2_D, max_seq, vb.NO_WINDOW)
    cache = vb.KvCache(ctx, C2_LAYERS, C2_HEADS, C2_D, max_seq, "f16")
    be = vb.HipAttentionBackend(ctx)
    outs = np.zeros((C2_STEPS, C2_LAYERS, C2_HEADS * C2_D), np.float32)
    try:
        for l in range(C2_LAYERS):
            k, v = _layer_kv(l)
            cache.write_rows("k", l, 0, np.ascontiguousarray(k).view(np.uint16))
            cache.write_rows("v", l, 0, np.ascontiguousarray(v).view(np.uint16))
        cache.pos = C2_L0
        bufs = []
        for s in range(C2_STEPS):
            io = []
            for l in range(C2_LAYERS):
                q, kc, vc = _step_inputs(l, s)
                io.append((ctx.to_device(q), ctx.to_device(kc), ctx.to_device(vc), ctx.alloc(q.nbytes)))
            bufs.append(io)
            vb.step_attention(be, cache, c, io)  # layer_step x 32, advance, finalize_token
            assert cache.pos == C2_L0 + s + 1
            for l in range(C2_LAYERS):
                outs[s, l] = ctx.download(io[l][3], np.float32, C2_HEADS * C2_D)
        # Appended rows: exactly the f32 -> f16 (nearest even) of k_cur / v_cur.
        for l in range(C2_LAYERS):
            got_k = cache.read_rows("k", l, max_seq)[C2_L0:]
            got_v = cache.read_rows("v", l, max_seq)[C2_L0:]
            for s in range(C2_STEPS):
                _, kc, vc = _step_inputs(l, s)
                assert np.array_equal(got_k[s].reshape(-1), orc.f32_to_f16_bits(kc)), f"layer {l} step {s}: K"
                assert np.array_equal(got_v[s].reshape(-1), orc.f32_to_f16_bits(vc)), f"layer {l} step {s}: V"
        # Stepping past max_seq raises KvCacheFull before any launch.
        with pytest.raises(vb.KvCacheFull):
            vb.step_attention(be, cache, c, bufs[0])
    finally:
        cache.close()
    pool = orc.Pool(16)
    try:
        oc = orc.OracleKvCache(1, C2_HEADS, C2_D, max_seq)
        cfg = orc.config(C2_HEADS, C2_HEADS, C2_D, max_seq)
        scores = np.zeros(C2_HEADS * max_seq, np.float32)
        for l in range(C2_LAYERS):
            k, v = _layer_kv(l)
            oc.layer_rows("k", 0)[:C2_L0] = k.astype(np.float32)
            oc.layer_rows("v", 0)[:C2_L0] = v.astype(np.float32)
            for s in range(C2_STEPS):
                q, kc, vc = _step_inputs(l, s)
                oc.layer_rows("k", 0)[C2_L0 + s] = kc.astype(np.float16).astype(np.float32).reshape(C2_HEADS, C2_D)
                oc.layer_rows("v", 0)[C2_L0 + s] = vc.astype(np.float16).astype(np.float32).reshape(C2_HEADS, C2_D)
                ref = pool.attention(q, oc, cfg, 0, C2_L0 + s, scores=scores)
                check(orc, outs[s, l], ref, C2_HEADS, "f16", what=f"C2 layer {l} step {s} (L={C2_L0 + s + 1})")
    finally:
        pool.close()


C2_FULL_STEPS = 256
C2_SAMPLED = (0, 1, 127, 255)


def test_c2_all_256_steps_sampled(ctx, orc):
    # BASELINE config 2 as written: 256 decode steps, the cache growing from
    # 4096 to 4352 rows, each step a layer_step per layer, one advance and
    # finalize_token (forward.zig:152-172, kv_cache.zig:130-133).
    import vantablack_amd as vb
    max_seq = C2_L0 + C2_FULL_STEPS
    c = vb.LlamaConfig(C2_HEADS, C2_HEADS, C2_D, max_seq, vb.NO_WINDOW)
    cache = vb.KvCache(ctx, C2_LAYERS, C2_HEADS, C2_D, max_seq, "f16")
    be = vb.HipAttentionBackend(ctx)
    n = C2_HEADS * C2_D
    outs = {s: np.zeros((C2_LAYERS, n), np.float32) for s in C2_SAMPLED}
    try:
        for l in range(C2_LAYERS):
            k, v = _layer_kv(l)
            cache.write_rows("k", l, 0, np.ascontiguousarray(k).view(np.uint16))
            cache.write_rows("v", l, 0, np.ascontiguousarray(v).view(np.uint16))
        cache.pos = C2_L0
        io = [(ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4 * n)) for _ in range(C2_LAYERS)]
        for s in range(C2_FULL_STEPS):
            for l in range(C2_LAYERS):
                for buf, arr in zip(io[l][:3], _step_inputs(l, s)):
                    ctx.upload(buf, arr)
            vb.step_attention(be, cache, c, io)
            assert cache.pos == C2_L0 + s + 1
            if s in outs:
                for l in range(C2_LAYERS):
                    outs[s][l] = ctx.download(io[l][3], np.float32, n)
        for l in range(C2_LAYERS):
            got_k = cache.read_rows("k", l, max_seq)[C2_L0:].reshape(C2_FULL_STEPS, n)
            got_v = cache.read_rows("v", l, max_seq)[C2_L0:].reshape(C2_FULL_STEPS, n)
            for s in range(C2_FULL_STEPS):
                _, kc, vc = _step_inputs(l, s)
                assert np.array_equal(got_k[s], orc.f32_to_f16_bits(kc)), f"layer {l} step {s}: K"
                assert np.array_equal(got_v[s], orc.f32_to_f16_bits(vc)), f"layer {l} step {s}: V"
        assert cache.pos == max_seq
    finally:
        cache.close()
    pool = orc.Pool(16)
    try:
        oc = orc.OracleKvCache(1, C2_HEADS, C2_D, max_seq)
        cfg = orc.config(C2_HEADS, C2_HEADS, C2_D, max_seq)
        scores = np.zeros(C2_HEADS * max_seq, np.float32)
        for l in range(C2_LAYERS):
            k, v = _layer_kv(l)
            oc.layer_rows("k", 0)[:C2_L0] = k.astype(np.float32)
            oc.layer_rows("v", 0)[:C2_L0] = v.astype(np.float32)
            for s in range(C2_FULL_STEPS):
                q, kc, vc = _step_inputs(l, s)
                oc.layer_rows("k", 0)[C2_L0 + s] = kc.astype(np.float16).astype(np.float32).reshape(C2_HEADS, C2_D)
                oc.layer_rows("v", 0)[C2_L0 + s] = vc.astype(np.float16).astype(np.float32).reshape(C2_HEADS, C2_D)
                if s in outs:
                    ref = pool.attention(q, oc, cfg, 0, C2_L0 + s, scores=scores)
                    check(orc, outs[s][l], ref, C2_HEADS, "f16", what=f"C2 256-step run: layer {l} step {s} "
                                                                        f"(L={C2_L0 + s + 1})")
    finally:
        pool.close()


def test_c5_decode_at_32768_bf16(ctx, orc):
    # BASELINE config 5 decode: 8 q heads, 1 KV head (MQA), d256, bf16 KV at
    # 32768 positions, the layer-level entry on layer 1 of two.
    err = decode_case(ctx, orc, 8, 1, 256, pos=32767, dtype="bf16", seed=55, q_scale=1.0 / 16.0, n_layers=2,
                      layer=1)
    print(f"C5 decode bf16 L=32768: rel err {err:.2e}")


def test_c3_decode_exact_point(ctx, orc):
    # 32/8 heads, d128, bf16, cache of 16384 rows, window
    # 4096 at position 16383 (window start 12288), 1% outlier channels x20.
    err = decode_case(ctx, orc, 32, 8, 128, pos=16383, dtype="bf16", window=4096, seed=33,
                      q_scale=1.0 / np.sqrt(128), outlier_frac=0.01, n_layers=2, layer=1)
    print(f"C3 decode bf16 window 4096 @16383: rel err {err:.2e}")
