"""Causal-prefill parity on the GPU, through the C ABI, against the oracle's
prefill.attentionCausal restatement.

The queries are f32 on both sides, as the reference's s.q is
(prefill.zig:167-197); only the cache rows carry the cache dtype.  Reduced
sizes are checked on every row; the BASELINE full sizes (C4 at 2048/8192
tokens, C5 at 4096) on every 8th row plus block and tile boundaries, with the
oracle's rows split over a pool.zig-style pool (parallel over heads), since
the oracle costs O(L) per row.
"""
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg
from tests.parity import check

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def prefill_case(ctx, orc, n_heads, n_kv, d, dtype, B, pos0=0, window=None, seed=0, rows=None,
                 extra_rows=0, k_scale=1.0, v_scale=1.0, q_scale=1.0, pooled=False):
    """Prefill B queries at positions pos0..pos0+B-1 over a cache of
    pos0 + B (+ extra_rows unwritten) rows, via vtb_hip_segment_attn_prefill.
    k_scale / v_scale / q_scale multiply the seeded N(0,1) inputs (a scalar,
    or an array broadcast over [rows, n_kv, d] / [B, n_heads*d]).  Returns
    the relative error against the oracle."""
    import vantablack_amd as vb
    n_rows = pos0 + B
    k = (orc.normal(seed * 10 + 1, n_rows * n_kv * d).reshape(n_rows, n_kv, d) * k_scale).astype(np.float32)
    v = (orc.normal(seed * 10 + 2, n_rows * n_kv * d).reshape(n_rows, n_kv, d) * v_scale).astype(np.float32)
    q = (orc.normal(seed * 10 + 3, B * n_heads * d).reshape(B, n_heads * d) * q_scale).astype(np.float32)
    ks, kx = orc.to_dtype(k, dtype)
    vs, vx = orc.to_dtype(v, dtype)
    pad = np.zeros((extra_rows, n_kv, d), ks.dtype)
    kb = ctx.to_device(np.concatenate([ks.reshape(n_rows, n_kv, d), pad]))
    vbuf = ctx.to_device(np.concatenate([vs.reshape(n_rows, n_kv, d), pad]))
    qb = ctx.to_device(q)
    ob = ctx.alloc(B * n_heads * d * 4)
    W = vb.NO_WINDOW if window is None else window
    with ctx.segment() as seg:
        seg.attn_prefill(ob, qb, kb, vbuf, 0, B, pos0, W, n_heads, n_kv, d, 1.0 / np.sqrt(d),
                         vb.hip.DTYPES[dtype])
    got = ctx.download(ob, np.float32, B * n_heads * d).reshape(B, n_heads * d)
    oc = orc.OracleKvCache(1, n_kv, d, n_rows + extra_rows)
    oc.layer_rows("k", 0)[:n_rows] = kx.reshape(n_rows, n_kv, d)
    oc.layer_rows("v", 0)[:n_rows] = vx.reshape(n_rows, n_kv, d)
    oc.pos = pos0
    rows = list(range(B)) if rows is None else sorted(set(r for r in rows if 0 <= r < B))
    cfg = orc.config(n_heads, n_kv, d, n_rows + extra_rows, orc.NO_WINDOW if window is None else window)
    if pooled:
        ref = pooled_rows(orc, q, oc, cfg, pos0, rows)
    else:
        ref = orc.attention_causal(q.reshape(-1), oc, cfg, 0, rows)
    return check(orc, got[rows], ref, n_heads, dtype, n_queries=len(rows),
                 what=f"prefill h{n_heads}/{n_kv} d{d} {dtype} B{B} pos0 {pos0} w{window}")


def pooled_rows(orc, q, oc, cfg, pos0, rows, workers=16):
    """attentionCausal for the listed rows, each split over heads on the
    oracle's pool (bit-identical to the single-threaded restatement)."""
    pool = orc.Pool(workers)
    try:
        out = np.zeros((len(rows), q.shape[1]), np.float32)
        scores = np.zeros(cfg.n_heads * cfg.max_seq, np.float32)
        for i, b in enumerate(rows):
            out[i] = pool.attention(q[b], oc, cfg, 0, pos0 + b, scores=scores)
        return out
    finally:
        pool.close()


@pytest.mark.parametrize("case", [c for c in mg.TINY if c[7] > 1], ids=[c[0] for c in mg.TINY if c[7] > 1])
def test_prefill_golden_fixture(ctx, orc, case):
    import vantablack_amd as vb
    name, n_heads, n_kv, d, dtype, n_rows, pos0, n_tok, window, seed = case
    q, _, ks, kx, vs, vx = mg.tiny_inputs(n_heads, n_kv, d, dtype, n_rows, n_tok, seed)
    ob = ctx.alloc(n_tok * n_heads * d * 4)
    with ctx.segment() as seg:
        seg.attn_prefill(ob, ctx.to_device(q), ctx.to_device(ks), ctx.to_device(vs), 0, n_tok, pos0,
                         vb.NO_WINDOW if window is None else window, n_heads, n_kv, d, 1.0 / np.sqrt(d),
                         vb.hip.DTYPES[dtype])
    got = ctx.download(ob, np.float32, n_tok * n_heads * d)
    ref = np.load(os.path.join(GOLD, f"{name}.npz"))["out"]
    check(orc, got, ref, n_heads, dtype, n_queries=n_tok, what=name)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("n_heads,n_kv,d,B", [
    (8, 2, 128, 300),    # C4-shaped GQA 4:1, ragged length
    (4, 1, 256, 200),    # C5-shaped MQA d256
    (4, 4, 64, 257),     # d64 MHA, one past two blocks
    (6, 4, 128, 129),    # uneven GQA map
])
def test_prefill_shapes(ctx, orc, dtype, n_heads, n_kv, d, B):
    prefill_case(ctx, orc, n_heads, n_kv, d, dtype, B, seed=B + d)


@pytest.mark.parametrize("B", [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129])
def test_prefill_lengths(ctx, orc, B):
    prefill_case(ctx, orc, 4, 2, 128, "bf16", B, seed=B)


@pytest.mark.parametrize("pos0,B,window", [(37, 100, None), (500, 130, None), (0, 300, 64), (100, 200, 96),
                                           (1000, 64, 256), (10, 150, 1)])
def test_prefill_offsets_and_windows(ctx, orc, pos0, B, window):
    prefill_case(ctx, orc, 4, 2, 128, "bf16", B, pos0=pos0, window=window, seed=pos0 + B)


def test_prefill_reads_no_rows_beyond_the_prompt(ctx, orc):
    # Rows past pos0 + B hold garbage-free zeros here, but the result must not
    # depend on them: compare against the same case with no extra rows.
    prefill_case(ctx, orc, 4, 2, 64, "f16", 70, pos0=5, extra_rows=100, seed=4)


def test_prefill_f32_cache_uses_exact_path(ctx, orc):
    # f32 caches run the exact f32 split-K kernel per query: 1e-5 parity.
    prefill_case(ctx, orc, 8, 2, 64, "f32", 150, pos0=20, window=48, seed=5)


def test_prefill_row_equals_decode(ctx, orc):
    """prefill.zig:21-23: prefill row b equals a single-token decode at
    position pos0 + b (here: the MFMA prefill vs the f32 decode kernel on
    the same bf16 cache)."""
    import vantablack_amd as vb
    n_heads, n_kv, d, B, pos0 = 8, 2, 128, 96, 10
    n_rows = pos0 + B
    k = orc.to_dtype(orc.normal(71, n_rows * n_kv * d), "bf16")[0]
    v = orc.to_dtype(orc.normal(72, n_rows * n_kv * d), "bf16")[0]
    q = orc.normal(73, B * n_heads * d)
    kb, vbuf = ctx.to_device(k), ctx.to_device(v)
    ob = ctx.alloc(B * n_heads * d * 4)
    with ctx.segment() as seg:
        seg.attn_prefill(ob, ctx.to_device(q), kb, vbuf, 0, B, pos0, vb.NO_WINDOW, n_heads, n_kv, d,
                         1.0 / np.sqrt(d), vb.BF16)
    pre = ctx.download(ob, np.float32, B * n_heads * d).reshape(B, -1)
    for b in (0, 1, 47, 95):
        qb = ctx.to_device(q.reshape(B, -1)[b])
        od = ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            seg.attn_decode(od, qb, kb, 0, vbuf, 0, n_heads, n_kv, d, pos0 + b + 1, 1.0 / np.sqrt(d), vb.BF16)
        dec = ctx.download(od, np.float32, n_heads * d)
        check(orc, pre[b], dec, n_heads, "bf16", what=f"row {b}")


def test_prefill_attention_layer_entry(ctx, orc):
    """prefill.zig:174-197 through vtb_hip_prefill_attention: f32 K/V rows are
    appended at pos..pos+B-1 (rounded to bf16), then causal attention of the
    f32 queries with a sliding window, against the oracle fed the same f32
    queries."""
    import vantablack_amd as vb
    n_heads, n_kv, d, B, pos0, W, n_layers, layer = 8, 2, 128, 80, 30, 64, 2, 1
    max_seq = 256
    rng_k = orc.normal(81, (pos0 + B) * n_kv * d).reshape(pos0 + B, n_kv, d)
    rng_v = orc.normal(82, (pos0 + B) * n_kv * d).reshape(pos0 + B, n_kv, d)
    q = orc.normal(83, B * n_heads * d)
    ks, kx = orc.to_dtype(rng_k, "bf16")
    vs, vx = orc.to_dtype(rng_v, "bf16")
    cache = vb.KvCache(ctx, n_layers, n_kv, d, max_seq, "bf16")
    try:
        cache.write_rows("k", layer, 0, ks.reshape(pos0 + B, n_kv, d)[:pos0])
        cache.write_rows("v", layer, 0, vs.reshape(pos0 + B, n_kv, d)[:pos0])
        cache.pos = pos0
        c = vb.LlamaConfig(n_heads, n_kv, d, max_seq, W)
        ob = ctx.alloc(B * n_heads * d * 4)
        with ctx.segment() as seg:
            vb.prefill_attention(seg, cache, c, layer, B, ctx.to_device(q), ctx.to_device(rng_k[pos0:]),
                                 ctx.to_device(rng_v[pos0:]), ob)
        got = ctx.download(ob, np.float32, B * n_heads * d)
        assert cache.pos == pos0  # the caller advances pos after all layers (prefill.zig:141)
        written = cache.read_rows("k", layer, pos0 + B)
        assert np.array_equal(written.reshape(-1), ks.reshape(-1))
        with pytest.raises(vb.KvCacheFull):
            with ctx.segment() as seg:
                vb.prefill_attention(seg, cache, c, layer, max_seq - pos0 + 1, ctx.to_device(q),
                                     ctx.to_device(rng_k), ctx.to_device(rng_v), ob)
    finally:
        cache.close()
    oc = orc.OracleKvCache(n_layers, n_kv, d, max_seq)
    oc.layer_rows("k", layer)[:pos0 + B] = kx.reshape(pos0 + B, n_kv, d)
    oc.layer_rows("v", layer)[:pos0 + B] = vx.reshape(pos0 + B, n_kv, d)
    oc.pos = pos0
    ref = orc.attention_causal(q, oc, orc.config(n_heads, n_kv, d, max_seq, W), layer, range(B))
    check(orc, got, ref, n_heads, "bf16", n_queries=B, what="prefill layer entry")


def test_prefill_scratch_growth_keeps_inputs_intact(ctx, orc):
    """Regression: growing the prefill scratch (layer-level prefill with a
    longer prompt) must leave inputs allocated afterwards untouched by
    repeated prefills, and repeats agree bit for bit."""
    import vantablack_amd as vb
    n_heads, n_kv, d = 8, 2, 128
    own = vb.Context()  # a fresh context: its scratch buffers start unallocated
    try:
        assert prefill_case(own, orc, n_heads, n_kv, d, "bf16", 64, seed=71) <= 2e-3  # scratch exists
        for B in (16, 200):  # the second call grows the scratch
            cache = vb.KvCache(own, 1, n_kv, d, 256, "bf16")
            try:
                c = vb.LlamaConfig(n_heads, n_kv, d, 256, vb.NO_WINDOW)
                kv = orc.normal(72, B * n_kv * d)
                with own.segment() as seg:
                    vb.prefill_attention(seg, cache, c, 0, B, own.to_device(orc.normal(73, B * n_heads * d)),
                                         own.to_device(kv), own.to_device(kv), own.alloc(B * n_heads * d * 4))
                own.wait_idle()
            finally:
                cache.close()
        B = 256
        vs = orc.to_dtype(orc.normal(74, B * n_kv * d), "bf16")[0]
        ks = orc.to_dtype(orc.normal(75, B * n_kv * d), "bf16")[0]
        qs = orc.normal(76, B * n_heads * d)
        vbuf, kb, qb = own.to_device(vs), own.to_device(ks), own.to_device(qs)
        outs = []
        for _ in range(3):
            ob = own.alloc(B * n_heads * d * 4)
            with own.segment() as seg:
                seg.attn_prefill(ob, qb, kb, vbuf, 0, B, 0, vb.NO_WINDOW, n_heads, n_kv, d, 1 / np.sqrt(d),
                                 vb.BF16)
            outs.append(own.download(ob, np.float32, B * n_heads * d))
        assert np.array_equal(own.download(vbuf, vs.dtype, vs.size), vs), "V input overwritten"
        assert np.array_equal(own.download(kb, ks.dtype, ks.size), ks), "K input overwritten"
        assert all(np.array_equal(outs[0], o) for o in outs[1:]), "repeated prefill differs"
        assert np.isfinite(outs[0]).all()
    finally:
        own.close()


def _dense_rows(B, stride, bm=256):
    """Every stride-th row plus the first, last and block / tile edges."""
    rows = set(range(0, B, stride)) | {1, B - 1, B - 2}
    for blk in range(1, B // bm + 1):
        rows |= {blk * bm - 1, blk * bm, blk * bm + 31, blk * bm + 32, blk * bm + 63, blk * bm + 64}
    return sorted(r for r in rows if 0 <= r < B)


@pytest.mark.parametrize("B", [512, 2048])
def test_c4_llama3_prefill_all_rows(ctx, orc, B):
    # 32 q heads, 8 KV heads, d128, bf16, causal, pos0 0;
    # f32 queries, every row against the oracle.
    prefill_case(ctx, orc, 32, 8, 128, "bf16", B, seed=400 + B, pooled=True)


def test_c4_llama3_prefill_8192(ctx, orc):
    prefill_case(ctx, orc, 32, 8, 128, "bf16", 8192, seed=400 + 8192, rows=_dense_rows(8192, 8), pooled=True)


def test_c5_gemma_prefill_full_size(ctx, orc):
    # BASELINE config 5 prefill: 8 q heads, 1 KV head (MQA), d256, bf16, 4096 tokens.
    prefill_case(ctx, orc, 8, 1, 256, "bf16", 4096, seed=500, rows=_dense_rows(4096, 4), pooled=True)


# Balanced pairs of query blocks (the d256 kernel): blocks b and c = nblk-1-b
# pair up, block c's keys are cut at the pair's midpoint over two
# workgroups and merged by whichever arrives second, and the first
# workgroup of the pair also takes block b whole.  Each shape runs paired
# (the default) and unpaired against the oracle: prompt offsets, a partial
# last block, one pair, and the two-piece precision path (large scores).
@pytest.mark.parametrize("balance", ["1", "0"])
@pytest.mark.parametrize("n_heads,B,pos0,q_scale", [
    (2, 512, 0, 1.0), (3, 1024, 0, 1.0), (2, 768, 300, 1.0), (1, 256, 37, 1.0), (2, 1000, 0, 1.0),
    (2, 512, 0, 8.0),
])
def test_prefill_d256_balanced_pairs(ctx, orc, monkeypatch, balance, n_heads, B, pos0, q_scale):
    monkeypatch.setenv("VTB_PREFILL_BALANCE", balance)
    err = prefill_case(ctx, orc, n_heads, 1, 256, "bf16", B, pos0=pos0, seed=900 + B, q_scale=q_scale)
    print(f"d256 balance={balance} h{n_heads} B{B} pos0 {pos0} q x{q_scale}: rel err {err:.2e}")


# Ranges beyond f16's: the pre-pass scales each bf16 head by a power of two
# (keys / values) and each wave's queries likewise, so magnitudes above 65504
# or below f16's normal range keep 11 significant bits.  Scores stay O(1)
# where one operand grows and the other shrinks, so the cases are as well
# conditioned as the N(0,1) ones.
@pytest.mark.parametrize("what,ks,vs,qs", [
    ("v_above_f16", 1.0, 3.0e5, 1.0),          # |v| up to ~1.5e6 > 65504
    ("v_below_f16", 1.0, 1.0e-7, 1.0),         # every |v| in f16's subnormal range
    ("k_above_q_below", 2.0e5, 1.0, 5.0e-6),   # |k| > 65504, tiny q
    ("q_above_k_below", 3.0e-6, 1.0, 4.0e5),   # |q| > 65504, tiny k
])
def test_prefill_range_beyond_f16(ctx, orc, what, ks, vs, qs):
    prefill_case(ctx, orc, 8, 2, 128, "bf16", 300, seed=77, k_scale=ks, v_scale=vs, q_scale=qs)


def test_prefill_v_outlier_rows_beyond_f16(ctx, orc):
    # A few V rows at ~1e6 among N(0,1) rows of the same heads (a per-head
    # scale keeps both within f16's 2^29 normal range).
    n_rows = 400
    scale = np.ones((n_rows, 2, 1), np.float32)
    scale[[5, 77, 301]] = 7.0e5
    prefill_case(ctx, orc, 8, 2, 128, "bf16", n_rows, seed=78, v_scale=scale)


# Value exponents per 64-key tile: bf16 value tiles whose ranges differ by
# 16x or more get their own power-of-two unit, and the attention rescales O
# whenever the unit changes (up the ramp, down it, through an all-zero tile
# that fits any unit), including the d256 balanced launches, whose two
# pieces of a split block then merge from different units.
def _tile_ramp(n_rows, step, zero_tile=None):
    sc = (2.0 ** (step * (np.arange(n_rows) // 64))).astype(np.float32).reshape(n_rows, 1, 1)
    if zero_tile is not None:
        sc[64 * zero_tile:64 * (zero_tile + 1)] = 0.0
    return sc


@pytest.mark.parametrize("what,step,zero_tile", [("ramp_up", 5.0, None), ("ramp_down", -5.0, None),
                                                   ("zero_tile", 0.0, 2), ("ramp_up_zero_tile", 3.0, 4)])
def test_prefill_value_tile_exponents(ctx, orc, what, step, zero_tile):
    n_rows = 520
    err = prefill_case(ctx, orc, 8, 2, 128, "bf16", n_rows, seed=83, v_scale=_tile_ramp(n_rows, step, zero_tile))
    print(f"value tiles {what}: rel err {err:.2e}")


@pytest.mark.parametrize("balance", ["1", "0"])
@pytest.mark.parametrize("step", [4.0, -4.0])
def test_prefill_d256_value_tile_exponents(ctx, orc, monkeypatch, balance, step):
    monkeypatch.setenv("VTB_PREFILL_BALANCE", balance)
    err = prefill_case(ctx, orc, 2, 1, 256, "bf16", 512, seed=84, v_scale=_tile_ramp(512, step))
    print(f"d256 value tiles step {step} balance={balance}: rel err {err:.2e}")


def test_prefill_pre_pass_starts_at_the_window(ctx, orc):
    # Keys before the first query's window start are never read: the
    # pre-pass starts at that key's 64-key tile and the attention's key loop
    # and statistics at each block's own window start.  Rows before that
    # tile hold NaN here (the oracle never reads them either); rows of that
    # tile before the window start are finite and masked.
    pos0, B, W = 1000, 100, 200
    n_rows = pos0 + B
    ks = np.ones((n_rows, 2, 1), np.float32)
    ks[:(pos0 - W + 1) // 64 * 64] = np.nan
    prefill_case(ctx, orc, 8, 2, 128, "bf16", B, pos0=pos0, window=W, seed=85, k_scale=ks, v_scale=ks)


# A work item takes q as two f16 pieces when the Cauchy-Schwarz bound on its
# scores (max |q| * max |k_t| * scale_log2 over its key tiles) exceeds 32,
# and P as two pieces when its values' crest factor (max / rms over those
# tiles) exceeds 8: with one piece each, x20 channel outliers (the C3
# recipe) measured 6.9e-3 against the oracle.  Every kernel shape holds all
# three compiled forms (q alone; q and P; neither).
@pytest.mark.parametrize("n_heads,n_kv,d,B", [
    (8, 2, 128, 333),   # d128 (two-piece path with K fragments read in halves)
    (8, 2, 64, 300),    # d64
    (4, 1, 256, 200),   # d256 (one wave per SIMD)
])
def test_prefill_channel_outliers_c3_style(ctx, orc, n_heads, n_kv, d, B):
    ch = np.ones((1, n_kv, d), np.float32)
    n_out = max(1, n_kv * d // 100)
    ch.reshape(-1)[np.random.default_rng(3).choice(n_kv * d, n_out, replace=False)] = 20.0
    err = prefill_case(ctx, orc, n_heads, n_kv, d, "bf16", B, seed=79, k_scale=ch, v_scale=ch)
    print(f"channel outliers h{n_heads}/{n_kv} d{d}: rel err {err:.2e}")


def test_prefill_mixed_heads_outliers_in_one_kv_head(ctx, orc):
    # One KV head with x20 channels, the other N(0,1): both paths in one
    # launch; f16 cache (no value scaling, the flags still apply).
    ch = np.ones((1, 2, 128), np.float32)
    ch[0, 1, [3, 77]] = 20.0
    prefill_case(ctx, orc, 8, 2, 128, "f16", 290, seed=81, k_scale=ch, v_scale=ch)


def test_prefill_range_beyond_f16_several_blocks(ctx, orc):
    # Five query blocks, the same per-head / per-wave scales.
    prefill_case(ctx, orc, 8, 2, 128, "bf16", 520, seed=80, v_scale=3.0e5, k_scale=2.0e5, q_scale=5.0e-6)


def test_prefill_large_scores_take_two_pieces(ctx, orc):
    # q and k of rms ~40: scores of ~1e3 (a one-hot softmax), where q's 11-bit
    # rounding alone would move a score by ~0.5; the score bound selects
    # two-piece q (values N(0,1): P in one piece).
    prefill_case(ctx, orc, 8, 2, 64, "bf16", 280, seed=82, k_scale=40.0, q_scale=40.0)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_prefill_large_scores_q_pieces_only_each_shape(ctx, orc, d):
    # The q-only form in every kernel shape: large scores, N(0,1) values.
    n_kv = 1 if d == 256 else 2
    prefill_case(ctx, orc, 4 * n_kv, n_kv, d, "f16", 300, seed=86, k_scale=12.0, q_scale=12.0)


def test_prefill_value_outliers_alone_take_p_pieces(ctx, orc):
    # Small scores, a few value rows x300 (crest far above 8): the P pieces
    # (compiled together with the q pieces).
    n_rows = 400
    vs = np.ones((n_rows, 2, 1), np.float32)
    vs[[9, 150, 390]] = 300.0
    prefill_case(ctx, orc, 8, 2, 128, "f16", n_rows, seed=87, v_scale=vs, q_scale=0.25)


# Key-split small-prompt form (d <= 128; launch_prefill_mfma picks it when
# 128-query workgroups would fill at most half the CUs): 64 queries per
# workgroup, two waves per 32 queries taking alternate key tiles, their
# partials merged through LDS as half 0's terms plus half 1's.  Each case
# runs forced on (VTB_PREFILL_KS=2) and off (=0) against the oracle: C4 at
# 512 tokens, a single query, one tile plus one key (the second half has no
# tile), offsets, a window that starts mid-prompt, MQA d64, an uneven GQA map,
# both two-piece precision forms (large scores; value outliers), and a long
# prompt where the key ranges run many steps.
@pytest.mark.parametrize("ks", ["2", "0"])
@pytest.mark.parametrize("n_heads,n_kv,d,dtype,B,pos0,window,q_scale,v_outliers", [
    (32, 8, 128, "bf16", 512, 0, None, 1.0, False),
    (8, 2, 128, "bf16", 1, 0, None, 1.0, False),
    (8, 2, 128, "bf16", 65, 0, None, 1.0, False),
    (8, 2, 128, "f16", 200, 37, None, 1.0, False),
    (8, 2, 128, "bf16", 300, 100, 96, 1.0, False),
    (8, 1, 64, "bf16", 333, 0, None, 1.0, False),
    (6, 4, 128, "bf16", 129, 0, None, 1.0, False),
    (8, 2, 128, "bf16", 256, 0, None, 8.0, False),
    (8, 2, 128, "bf16", 320, 0, None, 1.0, True),
    (4, 1, 128, "bf16", 1500, 20, None, 1.0, False),
])
def test_prefill_key_split(ctx, orc, monkeypatch, ks, n_heads, n_kv, d, dtype, B, pos0, window, q_scale,
                           v_outliers):
    monkeypatch.setenv("VTB_PREFILL_KS", ks)
    v_scale = 1.0
    if v_outliers:  # 1% of value channels x20: crest factor above 8 (P as two pieces)
        v_scale = np.ones((1, n_kv, d), np.float32)
        v_scale[:, :, ::97] = 20.0
    rows = None if B * n_heads <= 4096 else _dense_rows(B, 3, bm=64)
    err = prefill_case(ctx, orc, n_heads, n_kv, d, dtype, B, pos0=pos0, window=window, seed=1200 + B,
                       q_scale=q_scale, v_scale=v_scale, rows=rows, pooled=B * n_heads > 4096)
    print(f"key split={ks} h{n_heads}/{n_kv} d{d} {dtype} B{B} pos0 {pos0} w{window}: rel err {err:.2e}")
