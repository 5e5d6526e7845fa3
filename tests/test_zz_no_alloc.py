"""The no-allocation decode entry (vtb_hip_segment_attn_decode_append_noalloc)
against the allocating one (vtb_hip_segment_attn_decode_append) through the C
ABI: two calls in a row on the fixed scratch, the second with a smaller
input, each bit-identical to the existing entry on the same inputs (the same
kernels and split plan; only where the split-K workspace lives differs).
The no-allocation calls run first, on a fresh context, and the context's
growable scratch (split-K workspace, counters, prefill and matmul scratch)
must read zero bytes before and after them: a path that fell back on the
context workspace would grow it.
Also: a shape whose workspace exceeds the fixed scratch is rejected at commit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(orc, n_heads, n_kv, d, L, dtype, seed):
    rng = np.random.default_rng(seed)
    rows = L
    k = rng.standard_normal((rows, n_kv, d)).astype(np.float32)
    v = rng.standard_normal((rows, n_kv, d)).astype(np.float32)
    ks, _ = orc.to_dtype(k, dtype)
    vs, _ = orc.to_dtype(v, dtype)
    q = (rng.standard_normal(n_heads * d) / np.sqrt(d)).astype(np.float32)
    kc = rng.standard_normal(n_kv * d).astype(np.float32)
    vc = rng.standard_normal(n_kv * d).astype(np.float32)
    return ks, vs, q, kc, vc


def _run(c, inputs, n_heads, n_kv, d, L, dtype, noalloc):
    import vantablack_amd as vb
    ks, vs, q, kc, vc = inputs
    kb, vbuf = c.to_device(ks), c.to_device(vs)  # fresh caches: the fused append writes row L-1
    qb, kcb, vcb = c.to_device(q), c.to_device(kc), c.to_device(vc)
    ob = c.alloc(n_heads * d * 4)
    with c.segment() as seg:
        f = seg.attn_decode_append_noalloc if noalloc else seg.attn_decode_append
        f(ob, qb, kb, 0, vbuf, 0, kcb, vcb, n_heads, n_kv, d, L, 1.0 / np.sqrt(d), vb.hip.DTYPES[dtype])
    c.wait_idle()
    return c.download(ob, np.float32, n_heads * d)


# C2's head shape at 8K rows (8 splits per head), then a smaller GQA d256
# case (more splits, two-level merge) on the same fixed scratch.
CASES = ((32, 32, 128, 8193, "f16", 1), (8, 1, 256, 20000, "bf16", 2))


def test_noalloc_decode_matches_the_allocating_entry_twice(orc):
    # One fresh context for both entries: a context's split plan (its
    # per-XCD row weights, measured at init) fixes the summation order, so
    # the two entries agree bit for bit only on the same context.
    import vantablack_amd as vb
    inputs = [_inputs(orc, *args) for args in CASES]
    fresh = vb.Context()
    try:
        assert fresh.scratch_bytes == 0
        got = [_run(fresh, inp, *args[:5], noalloc=True) for inp, args in zip(inputs, CASES)]
        assert fresh.scratch_bytes == 0, "the no-allocation entry grew the context's workspace"
        for inp, args, b in zip(inputs, CASES, got):
            a = _run(fresh, inp, *args[:5], noalloc=False)
            assert np.isfinite(b).all()
            assert np.array_equal(a, b), f"noalloc differs from the allocating entry for {args}"
    finally:
        fresh.close()


def test_noalloc_decode_rejects_a_workspace_beyond_the_scratch(ctx, orc, monkeypatch):
    import vantablack_amd as vb
    # 4096 workgroups for 16 KV heads (GQA 4:1) of d256: 256 splits per
    # head, partials 16 x 256 x 4 x 258 x 4 B = 16.9 MB > 8 MiB.
    monkeypatch.setenv("VTB_DECODE_TARGET_WGS", "4096")
    n_heads, n_kv = 64, 16
    d, L = 256, 16384
    kb, vbuf = ctx.alloc(L * n_kv * d * 2), ctx.alloc(L * n_kv * d * 2)
    qb, ob = ctx.alloc(n_heads * d * 4), ctx.alloc(n_heads * d * 4)
    kcb, vcb = ctx.alloc(n_kv * d * 4), ctx.alloc(n_kv * d * 4)
    with pytest.raises(vb.HipError):
        with ctx.segment() as seg:
            seg.attn_decode_append_noalloc(ob, qb, kb, 0, vbuf, 0, kcb, vcb, n_heads, n_kv, d, L, 0.0625, vb.F16)
