"""Decode-attention parity on the GPU, through the C ABI, against the oracle.

Covers every BASELINE config's decode shape at parity size (C1 in full), the
dtypes f32/f16/bf16, GQA widths 1..16 including the uneven (h*n_kv)/n_heads
map, head_dim 64/128/256, the sliding window, and lengths at and around the
kernel's tile and split boundaries.
"""
import numpy as np
import pytest

from tests.parity import TOL, check, decode_case, make_kv
from tests.util import rel_err

pytestmark = pytest.mark.gpu


def test_c1_tinyllama_decode_f32(ctx, orc):
    # BASELINE config 1 exactly: 32 q heads, 4 KV heads, d64, f32 KV filled
    # to 512 positions, Q/K/V ~ N(0,1)/sqrt(64), seed 0.
    import vantablack_amd as vb
    n_heads, n_kv, d, L = 32, 4, 64, 512
    s = np.float32(1.0 / np.sqrt(d))
    k = (orc.normal(0, L * n_kv * d, offset=0) * s).reshape(L, n_kv, d)
    v = (orc.normal(0, L * n_kv * d, offset=L * n_kv * d) * s).reshape(L, n_kv, d)
    q = orc.normal(0, n_heads * d, offset=2 * L * n_kv * d) * s
    cache = vb.KvCache(ctx, 1, n_kv, d, L, "f32")
    try:
        cache.write_rows("k", 0, 0, k[:L - 1])
        cache.write_rows("v", 0, 0, v[:L - 1])
        cache.pos = L - 1
        c = vb.LlamaConfig(n_heads, n_kv, d, L)
        qb, kb, vbuf, ob = ctx.to_device(q), ctx.to_device(k[L - 1]), ctx.to_device(v[L - 1]), ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            vb.layer_attention(seg, cache, c, 0, qb, kb, vbuf, ob)
        got = ctx.download(ob, np.float32, n_heads * d)
    finally:
        cache.close()
    oc = orc.OracleKvCache(1, n_kv, d, L)
    oc.layer_rows("k", 0)[:] = k
    oc.layer_rows("v", 0)[:] = v
    oc.pos = L - 1
    ref = orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, L), 0)
    check(orc, got, ref, n_heads, "f32", what="C1")
    golden = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "c1_decode.npz"))
    assert rel_err(got, golden["out"], n_heads) <= 1e-5


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n_heads,n_kv,d", [
    (32, 32, 128),   # C2 MHA
    (32, 8, 128),    # C3 / C4 GQA 4:1
    (8, 1, 256),     # C5 MQA d256
    (32, 4, 64),     # C1 GQA 8:1
    (12, 4, 64),     # GQA 3:1 (template G=4 with a partial group)
    (6, 4, 128),     # uneven map: groups of 1 and 2
    (16, 1, 64),     # MQA 16:1 (widest template)
])
def test_decode_shapes(ctx, orc, dtype, n_heads, n_kv, d):
    decode_case(ctx, orc, n_heads, n_kv, d, pos=777, dtype=dtype, seed=n_heads + d)


@pytest.mark.parametrize("n_kv", [2, 8])
@pytest.mark.parametrize("pos", [0, 1, 2, 31, 32, 33, 127, 128, 129, 1023, 4095, 9000])
def test_decode_lengths(ctx, orc, pos, n_kv):
    # L = pos+1 runs through single-row, partial tiles, tile edges and many
    # splits, for GQA (n_kv 2) and MHA (n_kv 8: the row-major MHA kernel).
    decode_case(ctx, orc, 8, n_kv, 128, pos=pos, dtype="f16", seed=pos)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("pos,window", [(100, 4096), (4095, 4096), (4096, 4096), (5000, 4096), (300, 7), (40, 1)])
def test_decode_sliding_window(ctx, orc, dtype, pos, window):
    decode_case(ctx, orc, 32, 8, 128, pos=pos, dtype=dtype, window=window, seed=pos + window)


def test_decode_c3_outliers_bf16(ctx, orc):
    # C3 input distribution: 1% of K/V channels x20, window 4096, at parity size.
    decode_case(ctx, orc, 32, 8, 128, pos=6000, dtype="bf16", window=4096, seed=3, outlier_frac=0.01,
                q_scale=1.0 / np.sqrt(128))


def test_decode_nonzero_layer(ctx, orc):
    decode_case(ctx, orc, 8, 2, 64, pos=200, dtype="f32", n_layers=3, layer=2, max_seq=512, seed=9)


def test_sliding_window_known_answer(ctx):
    # forward.zig:297-364 on the device: 1 head, head_dim 2 is not a kernel
    # shape, so the same construction is embedded in head_dim 64 (extra dims 0).
    import vantablack_amd as vb
    d = 64
    cache = vb.KvCache(ctx, 1, 1, d, 8, "f32")
    try:
        K = np.zeros((6, 1, d), np.float32)
        V = np.zeros((6, 1, d), np.float32)
        for t in range(6):
            big = t < 3
            K[t, 0, 0] = 100.0 if big else 1.0
            V[t, 0, 0] = -999.0 if big else 1.0
        cache.write_rows("k", 0, 0, K[:5])
        cache.write_rows("v", 0, 0, V[:5])
        cache.pos = 5
        q = np.zeros(d, np.float32)
        q[0] = 1.0
        c = vb.LlamaConfig(1, 1, d, 8, sliding_window=3)
        ob = ctx.alloc(d * 4)
        with ctx.segment() as seg:
            vb.layer_attention(seg, cache, c, 0, ctx.to_device(q), ctx.to_device(K[5]), ctx.to_device(V[5]), ob)
        out = ctx.download(ob, np.float32, d)
    finally:
        cache.close()
    assert abs(out[0] - 1.0) <= 1e-3
    assert out[0] > -100.0


def test_split_count_independence(ctx, orc, monkeypatch):
    """The split-K merge is exact up to f32 rounding: any split count gives
    the same answer within the f32 tolerance, and a repeat run with the same
    split count is bit-identical (the arrival counters reset themselves)."""
    import vantablack_amd as vb
    n_heads, n_kv, d, L = 16, 4, 128, 3000
    ks, kx, vs, vx = make_kv(orc, L, n_kv, d, "f32", seed=5)
    q = orc.normal(6, n_heads * d)
    kb, vbuf, qb = ctx.to_device(ks), ctx.to_device(vs), ctx.to_device(q)
    outs = []
    for target in ("1", "16", "256", "4096", "4096"):
        monkeypatch.setenv("VTB_DECODE_TARGET_WGS", target)
        ob = ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            seg.attn_decode(ob, qb, kb, 0, vbuf, 0, n_heads, n_kv, d, L, 1.0 / np.sqrt(d), vb.F32)
        outs.append(ctx.download(ob, np.float32, n_heads * d))
    oc = orc.OracleKvCache(1, n_kv, d, L)
    oc.layer_rows("k", 0)[:] = kx
    oc.layer_rows("v", 0)[:] = vx
    oc.pos = L - 1
    ref = orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, L), 0)
    for o in outs:
        assert rel_err(o, ref, n_heads) <= TOL["f32"]
        assert rel_err(o, outs[0], n_heads) <= 5e-6
    assert np.array_equal(outs[3], outs[4])


def test_segment_decode_with_caller_window_offset(ctx, orc):
    """The bridge-level call: the caller shifts the K/V offset by window_start
    rows and passes attended_len (forward.zig:470-483)."""
    import vantablack_amd as vb
    n_heads, n_kv, d, pos, W = 8, 8, 128, 700, 256
    ks, kx, vs, vx = make_kv(orc, pos + 1, n_kv, d, "f16", seed=8)
    q = orc.normal(9, n_heads * d)
    ws = pos - W + 1
    row_bytes = n_kv * d * 2
    kb, vbuf, qb, ob = ctx.to_device(ks), ctx.to_device(vs), ctx.to_device(q), ctx.alloc(n_heads * d * 4)
    with ctx.segment() as seg:
        seg.attn_decode(ob, qb, kb, ws * row_bytes, vbuf, ws * row_bytes, n_heads, n_kv, d, W,
                        1.0 / np.sqrt(d), vb.F16)
    got = ctx.download(ob, np.float32, n_heads * d)
    oc = orc.OracleKvCache(1, n_kv, d, pos + 1)
    oc.layer_rows("k", 0)[:] = kx
    oc.layer_rows("v", 0)[:] = vx
    oc.pos = pos
    ref = orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, pos + 1, W), 0)
    check(orc, got, ref, n_heads, "f16", what="caller-window")


def test_decode_empty_sequence_zeroes_output(ctx):
    import vantablack_amd as vb
    ob = ctx.to_device(np.full(64 * 2, 7.0, np.float32))
    kb = ctx.alloc(1024)
    with ctx.segment() as seg:
        seg.attn_decode(ob, ctx.to_device(np.ones(128, np.float32)), kb, 0, kb, 0, 2, 1, 64, 0, 0.125, vb.F32)
    assert np.all(ctx.download(ob, np.float32, 128) == 0.0)


def test_bad_arguments_are_reported(ctx):
    import vantablack_amd as vb
    ob = ctx.alloc(4096)
    kb = ctx.alloc(4096)
    seg = ctx.segment()
    seg.attn_decode(ob, ob, kb, 0, kb, 0, 2, 1, 96, 4, 0.1, vb.F32)  # head_dim 96 unsupported
    with pytest.raises(vb.HipError) as e:
        seg.commit()
    assert e.value.rc == 5
    seg = ctx.segment()
    seg.attn_decode(ob, ob, kb, 0, kb, 0, 4, 1, 128, 4000, 0.1, vb.F32)  # K/V range past the buffer
    with pytest.raises(vb.HipError) as e:
        seg.commit()
    assert e.value.rc == 1


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_fused_append_matches_separate_calls(ctx, orc, dtype):
    """vtb_hip_segment_attn_decode_append == kv_append(K) + kv_append(V) +
    attn_decode, bit for bit, for both the output and the cache contents."""
    import vantablack_amd as vb
    n_heads, n_kv, d, L = 16, 4, 128, 2500
    ks, kx, vs, vx = make_kv(orc, L, n_kv, d, dtype, seed=12)
    q = orc.normal(13, n_heads * d)
    k_new, v_new = orc.normal(14, n_kv * d), orc.normal(15, n_kv * d)
    dt = vb.hip.DTYPES[dtype]
    row = n_kv * d * (4 if dtype == "f32" else 2)
    outs, caches = [], []
    for fused in (False, True):
        kb, vbuf = ctx.to_device(ks), ctx.to_device(vs)
        qb, kn, vn, ob = ctx.to_device(q), ctx.to_device(k_new), ctx.to_device(v_new), ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            if fused:
                seg.attn_decode_append(ob, qb, kb, 0, vbuf, 0, kn, vn, n_heads, n_kv, d, L, 1.0 / np.sqrt(d), dt)
            else:
                seg.kv_append(kb, (L - 1) * row, dt, kn, 0, n_kv * d)
                seg.kv_append(vbuf, (L - 1) * row, dt, vn, 0, n_kv * d)
                seg.attn_decode(ob, qb, kb, 0, vbuf, 0, n_heads, n_kv, d, L, 1.0 / np.sqrt(d), dt)
        outs.append(ctx.download(ob, np.float32, n_heads * d))
        npd = np.float32 if dtype == "f32" else np.uint16
        caches.append((ctx.download(kb, npd, L * n_kv * d), ctx.download(vbuf, npd, L * n_kv * d)))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])
    # and against the oracle with the appended row in place
    kx2, vx2 = kx.copy(), vx.copy()
    kx2[L - 1] = orc.to_dtype(k_new, dtype)[1].reshape(n_kv, d)
    vx2[L - 1] = orc.to_dtype(v_new, dtype)[1].reshape(n_kv, d)
    oc = orc.OracleKvCache(1, n_kv, d, L)
    oc.layer_rows("k", 0)[:] = kx2
    oc.layer_rows("v", 0)[:] = vx2
    oc.pos = L - 1
    check(orc, outs[1], orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, L), 0), n_heads, dtype,
          what="fused append")


@pytest.mark.parametrize("n_heads,n_kv,d,dtype,pos,target", [
    (8, 1, 256, "bf16", 32767, "256"),   # C5: 256 splits
    (12, 4, 64, "f16", 3000, "512"),     # partial GQA group (slots past the group), 128 splits
    (32, 32, 128, "f16", 8192, "1024"),  # head pairs, 64 splits
    (6, 4, 128, "f32", 2000, "600"),     # uneven GQA map, scalar form
])
def test_merge_launch_matches_in_kernel_merge(ctx, orc, monkeypatch, n_heads, n_kv, d, dtype, pos, target):
    """Merges of more splits than one level takes run as a launch of their
    own (vtb_decode_merge); against the oracle and against the in-kernel
    two-level merge of the same partials (a different but fixed summation
    order), each bit-identical when repeated."""
    import vantablack_amd as vb
    ks, kx, vs, vx = make_kv(orc, pos + 1, n_kv, d, dtype, seed=pos % 89)
    q = orc.normal(pos % 83 + 2, n_heads * d)
    kb, vbuf, qb = ctx.to_device(ks), ctx.to_device(vs), ctx.to_device(q)
    monkeypatch.setenv("VTB_DECODE_TARGET_WGS", target)
    oc = orc.OracleKvCache(1, n_kv, d, pos + 1)
    oc.layer_rows("k", 0)[:] = kx
    oc.layer_rows("v", 0)[:] = vx
    oc.pos = pos
    ref = orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, pos + 1), 0)
    got = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("VTB_DECODE_MERGE_LAUNCH", mode)
        outs = []
        for _ in range(2):
            ob = ctx.alloc(n_heads * d * 4)
            with ctx.segment() as seg:
                seg.attn_decode(ob, qb, kb, 0, vbuf, 0, n_heads, n_kv, d, pos + 1, 1.0 / np.sqrt(d),
                                vb.hip.DTYPES[dtype])
            outs.append(ctx.download(ob, np.float32, n_heads * d))
        assert np.array_equal(outs[0], outs[1])
        check(orc, outs[0], ref, n_heads, dtype, what=f"merge launch={mode} h{n_heads}/{n_kv} d{d} L{pos + 1}")
        got[mode] = outs[0]
    assert rel_err(got["1"], got["0"], n_heads) <= 2e-6


@pytest.mark.parametrize("pos", [1023, 1024])
def test_short_range_plan_boundary(ctx, orc, monkeypatch, pos):
    """C1's head shape (32/4 heads, f32, d64) at 256 workgroups: 1024 rows
    plan 32 splits of 32 rows with the flat in-kernel merge (the short-range
    rule), 1025 rows 52 splits of 20 rows and the merge launch.  Both against
    the oracle, each bit-identical when repeated."""
    import vantablack_amd as vb
    n_heads, n_kv, d = 32, 4, 64
    monkeypatch.setenv("VTB_DECODE_TARGET_WGS", "256")
    ks, kx, vs, vx = make_kv(orc, pos + 1, n_kv, d, "f32", seed=pos % 97)
    q = orc.normal(pos % 89 + 3, n_heads * d)
    kb, vbuf, qb = ctx.to_device(ks), ctx.to_device(vs), ctx.to_device(q)
    oc = orc.OracleKvCache(1, n_kv, d, pos + 1)
    oc.layer_rows("k", 0)[:] = kx
    oc.layer_rows("v", 0)[:] = vx
    oc.pos = pos
    ref = orc.cpu_attention(q, oc, orc.config(n_heads, n_kv, d, pos + 1), 0)
    outs = []
    for _ in range(2):
        ob = ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            seg.attn_decode(ob, qb, kb, 0, vbuf, 0, n_heads, n_kv, d, pos + 1, 1.0 / np.sqrt(d), vb.F32)
        outs.append(ctx.download(ob, np.float32, n_heads * d))
    assert np.array_equal(outs[0], outs[1])
    check(orc, outs[0], ref, n_heads, "f32", what=f"short-range plan L{pos + 1}")
