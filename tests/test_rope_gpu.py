"""Fused RoPE + KV-append + decode attention on the GPU, through the C ABI,
against the oracle: math.rope / math.ropeHalf (src/kernels/math.zig:85-133) of
q and k_cur at the position, the slot write, forward.cpuAttention
(forward.zig:250-270).  Same tolerances as every decode test (tests/parity.py).

The appended K row is compared with the oracle's rotated row rounded to the
cache dtype (sin/cos may differ from the host libm by an ulp, so the check
is a tolerance, and at most a rounding step for f16/bf16); the V row must land
bit-exactly.  At position 0 the rotation is exactly the identity, so the fused
path must equal the unrotated one bit for bit.
"""
import numpy as np
import pytest

from tests.parity import check, make_kv
from tests.util import rel_err

pytestmark = pytest.mark.gpu

ROW_TOL = {"f32": 2e-6, "f16": 1e-3, "bf16": 8e-3}


def _oracle(orc, q_rot, kx_hist, k_row, vx_hist, v_row, n_heads, n_kv, d, pos, window, f64=False):
    max_seq = pos + 1
    oc = orc.OracleKvCache(1, n_kv, d, max_seq)
    oc.layer_rows("k", 0)[:pos] = kx_hist
    oc.layer_rows("v", 0)[:pos] = vx_hist
    oc.layer_rows("k", 0)[pos] = k_row
    oc.layer_rows("v", 0)[pos] = v_row
    oc.pos = pos
    cfg = orc.config(n_heads, n_kv, d, max_seq, window)
    ref = orc.cpu_attention(q_rot, oc, cfg, 0)
    return (ref, orc.attention_f64(q_rot, oc, cfg, 0, pos)) if f64 else ref


def rope_case(ctx, orc, n_heads, n_kv, d, pos, dtype, half, base=10000.0, window=None, seed=0, f64=False):
    import vantablack_amd as vb
    W = orc.NO_WINDOW if window is None else window
    ks, kx, vs, vx = make_kv(orc, pos + 1, n_kv, d, dtype, seed)
    q = orc.normal(seed + 1000, n_heads * d)
    k_cur = orc.normal(seed + 2000, n_kv * d)          # f32, not yet rotated
    v_cur = vx[pos].reshape(-1).copy()
    cache = vb.KvCache(ctx, 1, n_kv, d, pos + 1, dtype)
    try:
        if pos > 0:
            cache.write_rows("k", 0, 0, ks[:pos])
            cache.write_rows("v", 0, 0, vs[:pos])
        cache.pos = pos
        c = vb.LlamaConfig(n_heads, n_kv, d, pos + 1, W, rope_base=base, rope_half=half)
        qb, kb, vb_, ob = ctx.to_device(q), ctx.to_device(k_cur), ctx.to_device(v_cur), ctx.alloc(n_heads * d * 4)
        with ctx.segment() as seg:
            vb.layer_attention_rope(seg, cache, c, 0, qb, kb, vb_, ob)
        ctx.wait_idle()
        got = ctx.download(ob, np.float32, n_heads * d)
        k_got = cache.read_rows("k", 0, pos + 1)[pos].reshape(-1)
        v_got = cache.read_rows("v", 0, pos + 1)[pos].reshape(-1)
        # q and k_cur are read, not rotated in place
        assert np.array_equal(ctx.download(qb, np.float32, n_heads * d), q)
        assert np.array_equal(ctx.download(kb, np.float32, n_kv * d), k_cur)
    finally:
        cache.close()
    q_rot = orc.rope(q.reshape(n_heads, d), pos, base, half=half).reshape(-1)
    k_rot = orc.rope(k_cur.reshape(n_kv, d), pos, base, half=half).reshape(-1)
    k_store, k_exact = orc.to_dtype(k_rot, dtype)
    # appended rows
    assert np.array_equal(v_got, vs[pos].reshape(-1)), "V slot write mismatch"
    k_got_f = {"f32": lambda b: b, "f16": orc.f16_bits_to_f32, "bf16": orc.bf16_bits_to_f32}[dtype](k_got)
    kerr = float(np.max(np.abs(k_got_f.astype(np.float64) - k_exact)) / np.max(np.abs(k_exact)))
    assert kerr <= ROW_TOL[dtype], f"rotated K row rel err {kerr:.2e}"
    what = f"rope decode h{n_heads}/{n_kv} d{d} pos{pos} {dtype} half{half} base{base} w{window}"
    if f64:
        return got, _oracle(orc, q_rot, kx[:pos], k_exact.reshape(n_kv, d), vx[:pos], vx[pos], n_heads, n_kv, d,
                            pos, W, f64=True)
    ref = _oracle(orc, q_rot, kx[:pos], k_exact.reshape(n_kv, d), vx[:pos], vx[pos], n_heads, n_kv, d, pos, W)
    return check(orc, got, ref, n_heads, dtype, what=what)


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n_heads,n_kv,d", [
    (32, 32, 128),   # C2 MHA
    (32, 8, 128),    # C3 GQA 4:1
    (8, 1, 256),     # C5 MQA d256
    (32, 4, 64),     # C1 GQA 8:1
    (6, 4, 128),     # uneven GQA map
])
def test_rope_decode_shapes(ctx, orc, dtype, half, n_heads, n_kv, d):
    rope_case(ctx, orc, n_heads, n_kv, d, pos=777, dtype=dtype, half=half, seed=n_heads + d)


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("pos,base", [(1, 10000.0), (2, 10000.0), (4095, 500000.0), (30000, 1000000.0),
                                      (30000, 10000.0)])
def test_rope_decode_positions_and_bases(ctx, orc, pos, base, half):
    # Large positions: the angle pos * inv_freq is formed from the same f32
    # table on both sides, so only sin/cos ulps separate them.  A 512-row
    # window keeps the f32 softmax short (see the long-context test below).
    rope_case(ctx, orc, 8, 1, 256, pos=pos, dtype="f32", half=half, base=base, window=512, seed=pos)


@pytest.mark.parametrize("half", [False, True])
def test_rope_long_f32_context_against_f64(ctx, orc, half):
    # 30001 attended f32 rows: the oracle's own sequential f32 sums carry
    # about sqrt(L) * 2^-24 ~ 1e-5 of relative error here, the size of the
    # f32 bar, so at this length both sides are held to the f64 formula:
    # the GPU must be within 1e-5 of it, and no further from it than the
    # f32 restatement is (plus 2e-6).
    got, (ref32, ref64) = rope_case(ctx, orc, 8, 1, 256, pos=30000, dtype="f32", half=half, base=1000000.0,
                                    seed=30000, f64=True)
    e_gpu = rel_err(got, ref64, 8)
    e_orc = rel_err(ref32, ref64, 8)
    assert e_gpu <= 1e-5, f"GPU vs f64 {e_gpu:.2e} (f32 oracle vs f64 {e_orc:.2e})"
    assert e_gpu <= e_orc + 2e-6, f"GPU vs f64 {e_gpu:.2e} > f32 oracle vs f64 {e_orc:.2e}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rope_decode_sliding_window(ctx, orc, dtype):
    # C3 shape: window 4096 at pos 16383 -- the rotation uses the absolute
    # position while the attention sees only the window.
    rope_case(ctx, orc, 32, 8, 128, pos=16383, dtype=dtype, half=False, window=4096, seed=7)


@pytest.mark.parametrize("half", [False, True])
def test_rope_pos0_equals_unrotated(ctx, orc, half):
    import vantablack_amd as vb
    n_heads, n_kv, d = 32, 8, 128
    q = orc.normal(5, n_heads * d)
    k_cur, v_cur = orc.normal(6, n_kv * d), orc.normal(7, n_kv * d)
    outs = []
    for rope in (False, True):
        cache = vb.KvCache(ctx, 1, n_kv, d, 16, "f16")
        try:
            cache.pos = 0
            c = vb.LlamaConfig(n_heads, n_kv, d, 16, rope_half=half)
            qb, kb, vb_, ob = ctx.to_device(q), ctx.to_device(k_cur), ctx.to_device(v_cur), ctx.alloc(n_heads * d * 4)
            backend = vb.HipAttentionBackend(ctx)
            backend.layer_step(cache, c, 0, qb, kb, vb_, ob, rope=rope)
            backend.finalize_token()
            outs.append((ctx.download(ob, np.float32, n_heads * d), cache.read_rows("k", 0, 1)))
        finally:
            cache.close()
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("half", [False, True])
def test_rope_segment_entry_windowed_view(ctx, orc, half):
    # The segment entry with the caller's window shift (forward.zig:470-483):
    # the K/V views start at window_start and seq_len is the attended length,
    # while RoPE uses the absolute position.
    import vantablack_amd as vb
    n_heads, n_kv, d, pos, window, base = 32, 8, 128, 5000, 1024, 500000.0
    ks, kx, vs, vx = make_kv(orc, pos + 1, n_kv, d, "bf16", 11)
    q = orc.normal(12, n_heads * d)
    k_cur = orc.normal(13, n_kv * d)
    v_cur = vx[pos].reshape(-1).copy()
    ws = pos - window + 1
    row_bytes = n_kv * d * 2
    kbuf = ctx.to_device(ks.reshape(-1))
    vbuf = ctx.to_device(vs.reshape(-1))
    qb, kb, vb_, ob = ctx.to_device(q), ctx.to_device(k_cur), ctx.to_device(v_cur), ctx.alloc(n_heads * d * 4)
    with ctx.segment() as seg:
        seg.attn_decode_rope_append(ob, qb, kbuf, ws * row_bytes, vbuf, ws * row_bytes, kb, vb_, n_heads, n_kv, d,
                                    window, float(1.0 / np.sqrt(d)), vb.BF16, pos, base, half)
    ctx.wait_idle()
    got = ctx.download(ob, np.float32, n_heads * d)
    q_rot = orc.rope(q.reshape(n_heads, d), pos, base, half=half).reshape(-1)
    k_rot = orc.rope(k_cur.reshape(n_kv, d), pos, base, half=half)
    _, k_exact = orc.to_dtype(k_rot, "bf16")
    ref = _oracle(orc, q_rot, kx[:pos], k_exact.reshape(n_kv, d), vx[:pos], vx[pos], n_heads, n_kv, d, pos, window)
    check(orc, got, ref, n_heads, "bf16", what="rope segment windowed")


def test_rope_rejects_bad_base(ctx):
    import vantablack_amd as vb
    n_heads, n_kv, d = 8, 8, 64
    cache = vb.KvCache(ctx, 1, n_kv, d, 4, "f32")
    try:
        cache.pos = 1
        c = vb.LlamaConfig(n_heads, n_kv, d, 4, rope_base=0.0)
        bufs = [ctx.alloc(n_heads * d * 4) for _ in range(4)]
        with pytest.raises(vb.HipError):
            with ctx.segment() as seg:
                vb.layer_attention_rope(seg, cache, c, 0, *bufs)
    finally:
        cache.close()
