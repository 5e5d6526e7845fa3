"""vtb_hip_reserve (the counterpart of prefill.zig Scratch.init,
prefill.zig:67-88): after one reservation, every decode range length,
prefill shape and batched-matmul size within its bounds runs without growing
the context's scratch, and gives bit-identical results to a context that
grew its scratch on demand."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, KVH, D = 32, 8, 128


def _run_all(ctx, dtype, max_seq, max_batch, k_mm, window, check=None):
    """Every decode length 1..max_seq, prefill shapes up to max_batch queries
    at the largest start, a fused-RoPE decode and a batched matmul; returns
    the outputs.  check() runs after each group of launches."""
    import vantablack_amd as vb
    rng = np.random.default_rng(7)
    dt = vb.hip.DTYPES[dtype]
    row = KVH * D
    kv_host = rng.standard_normal((max_seq, row)).astype(np.float32)
    if dtype == "f32":
        kv_bits = kv_host
    elif dtype == "f16":
        kv_bits = kv_host.astype(np.float16).view(np.uint16)
    else:
        kv_bits = (kv_host.view(np.uint32) >> 16).astype(np.uint16)
    k = ctx.to_device(kv_bits)
    v = ctx.to_device(kv_bits[::-1].copy())
    q = ctx.to_device(rng.standard_normal(max_batch * H * D).astype(np.float32))
    cur = ctx.to_device(rng.standard_normal(row).astype(np.float32))
    out = ctx.alloc(max_batch * H * D * 4)
    outs = []
    inv = 1.0 / np.sqrt(D)
    # Decode over every range length (the split plan changes with it).
    for L in range(1, max_seq + 1):
        with ctx.segment() as seg:
            seg.attn_decode(out, q, k, 0, v, 0, H, KVH, D, L, inv, dt)
        if L % 97 == 0 or L == max_seq:
            ctx.wait_idle()
            outs.append(ctx.download(out, np.float32, H * D))
    if check:
        check("decode")
    # Decode with the fused append + RoPE at the last slot, on copies.
    k2 = ctx.to_device(kv_bits)
    v2 = ctx.to_device(kv_bits)
    with ctx.segment() as seg:
        seg.attn_decode_rope_append(out, q, k2, 0, v2, 0, cur, cur, H, KVH, D, max_seq, inv, dt, max_seq - 1,
                                    10000.0)
    ctx.wait_idle()
    outs.append(ctx.download(out, np.float32, H * D))
    if check:
        check("decode_rope_append")
    # Prefill: query counts up to max_batch, starting where the context ends.
    for n in sorted({1, 2, 3, 17, 64, 65, max_batch // 2 + 1, max_batch}):
        pos0 = max_seq - n
        with ctx.segment() as seg:
            seg.attn_prefill(out, q, k, v, 0, n, pos0, window, H, KVH, D, inv, dt)
        ctx.wait_idle()
        outs.append(ctx.download(out, np.float32, n * H * D))
    if check:
        check("prefill")
    # Batched q8_0 matmul of max_batch tokens of width k_mm (zero-scale
    # blocks: the output is zero; the scratch is what is checked).
    m = 128
    w = ctx.to_device(np.zeros(m * (k_mm // 32) * 34, np.uint8))
    acts = ctx.to_device(rng.standard_normal(max_batch * k_mm).astype(np.float32))
    mo = ctx.alloc(max_batch * m * 4)
    for B in (1, max_batch // 3 + 1, max_batch):
        with ctx.segment() as seg:
            seg.matmul_batched("q8_0", mo, w, 0, acts, m, k_mm, B)
        ctx.wait_idle()
        outs.append(ctx.download(mo, np.float32, B * m))
    if check:
        check("matmul_batched")
    return outs


@pytest.mark.parametrize("dtype,window", [("bf16", None), ("f16", 300), ("f32", None)])
def test_reserve_covers_every_shape_within_bounds(dtype, window):
    import vantablack_amd as vb
    max_seq = 1024 if dtype != "f32" else 512
    max_batch, k_mm = 256, 2048
    w = vb.NO_WINDOW if window is None else window
    cfg = vb.LlamaConfig(H, KVH, D, max_seq, w)
    a = vb.Context()
    try:
        a.reserve(cfg.c(), dtype, max_batch, k_mm, 10000.0)
        reserved = a.scratch_bytes
        assert reserved > 0

        def check(what):
            assert a.scratch_bytes == reserved, f"{what} grew the reserved scratch"

        got = _run_all(a, dtype, max_seq, max_batch, k_mm, w, check)
    finally:
        a.close()
    b = vb.Context()
    try:
        want = _run_all(b, dtype, max_seq, max_batch, k_mm, w)
    finally:
        b.close()
    assert len(got) == len(want)
    for g, r in zip(got, want):
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32))


def test_reserve_rejects_out_of_range_bounds(ctx):
    import vantablack_amd as vb
    cfg = vb.LlamaConfig(H, KVH, D, 64)
    with pytest.raises(vb.HipError) as e:
        ctx.reserve(cfg.c(), "bf16", 65)
    assert e.value.rc == vb.hip.EUNSUPPORTED
    with pytest.raises(vb.HipError) as e:
        ctx.reserve(cfg.c(), "bf16", 16, 65536)
    assert e.value.rc == vb.hip.EUNSUPPORTED
    with pytest.raises(vb.HipError) as e:
        ctx.reserve(vb.LlamaConfig(H, KVH, 96, 64).c(), "bf16", 16)
    assert e.value.rc == vb.hip.EUNSUPPORTED
