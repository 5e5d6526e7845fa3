"""Full-GPU decode layer through the C ABI: the four layer ops
(vtb_hip_segment_rmsnorm / swiglu / gelu_approx / residual_add) against the
oracle's restatements of math.zig, then a small quantised model decoded token
by token with vantablack_amd.layer (the host side of gpuLayerStep,
forward.zig:419-513, and gpuFinalStep, :515-520) against oracle.cpu_layer_step
(cpuLayerStep, forward.zig:230-288), down to the argmax of the logits.

Bars: the ops hold 2e-6 of the largest reference value (residual_add exact);
the model's residual stream and logits hold 1e-4 of their largest value
after the layers (f32 throughout, summation orders differ), and the logits'
argmax agrees unless the reference's top two are within that bar.
"""
import numpy as np
import pytest

from tests.quant import random_weights

pytestmark = pytest.mark.gpu


def _views(ctx, arr, unaligned):
    """arr on the device as a Buffer whose base is 16-byte aligned, or 4 bytes
    past that (a view into a larger allocation); returns (view, backing)."""
    back = ctx.to_device(np.concatenate([np.zeros(1, np.float32), arr]) if unaligned else arr)
    if not unaligned:
        return back, back
    return ctx.wrap(back.ptr + 4, arr.nbytes, keepalive=back), back


@pytest.mark.parametrize("unaligned", [False, True])
@pytest.mark.parametrize("n", [1, 5, 4096, 5003])
def test_rmsnorm(ctx, orc, n, unaligned):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    xb, _ = _views(ctx, x, unaligned)
    wpad = np.concatenate([np.zeros(1 if unaligned else 4, np.float32), w])
    wb = ctx.to_device(wpad)
    ob, oback = _views(ctx, np.zeros(n, np.float32), unaligned)
    with ctx.segment() as seg:
        seg.rmsnorm(ob, xb, wb, (1 if unaligned else 4) * 4, n, 1e-5)
    ctx.wait_idle()
    got = ctx.download(oback, np.float32, n, offset=4 if unaligned else 0)
    ref = orc.rms_norm(x, w, 1e-5)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_rmsnorm_in_place(ctx, orc):
    # gpuFinalStep normalises x into itself (forward.zig:517).
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.random(4096).astype(np.float32)
    xb, wb = ctx.to_device(x), ctx.to_device(w)
    with ctx.segment() as seg:
        seg.rmsnorm(xb, xb, wb, 0, 4096, 1e-6)
    got = ctx.download(xb, np.float32, 4096)
    ref = orc.rms_norm(x, w, 1e-6)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


@pytest.mark.parametrize("unaligned", [False, True])
@pytest.mark.parametrize("n", [1, 3, 1000, 4099])
@pytest.mark.parametrize("op", ["swiglu", "gelu_approx", "residual_add"])
def test_elementwise_ops(ctx, orc, op, n, unaligned):
    rng = np.random.default_rng(n + len(op))
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    gb, gback = _views(ctx, g, unaligned)
    ub, _ = _views(ctx, u, unaligned)
    with ctx.segment() as seg:
        getattr(seg, op)(gb, ub, n)
    ctx.wait_idle()
    got = ctx.download(gback, np.float32, n, offset=4 if unaligned else 0)
    if op == "residual_add":
        assert np.array_equal(got, g + u)
        return
    ref = orc.swiglu(g, u) if op == "swiglu" else orc.geglu_approx(g, u)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("unaligned", [False, True])
@pytest.mark.parametrize("n", [3, 4096, 5003])
def test_residual_add_rmsnorm(ctx, orc, n, unaligned, in_place):
    # x += b, then out = rmsnorm(x) * w: the two ops back to back, in one launch.
    rng = np.random.default_rng(n + 17)
    x = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    xv, xback = _views(ctx, x, unaligned)
    bv, _ = _views(ctx, b, unaligned)
    wb = ctx.to_device(w)
    ov, oback = (xv, xback) if in_place else _views(ctx, np.zeros(n, np.float32), unaligned)
    with ctx.segment() as seg:
        seg.residual_add_rmsnorm(xv, bv, ov, wb, 0, n, 1e-5)
    ctx.wait_idle()
    off = 4 if unaligned else 0
    ref = orc.rms_norm(x + b, w, 1e-5)
    got = ctx.download(oback, np.float32, n, offset=off)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))
    if not in_place:
        assert np.array_equal(ctx.download(xback, np.float32, n, offset=off), x + b)


def test_ops_reject_ranges_beyond_the_buffer(ctx):
    import vantablack_amd as vb
    a, b = ctx.alloc(64), ctx.alloc(1024)
    for call in (lambda s: s.rmsnorm(a, b, b, 0, 32, 1e-5), lambda s: s.rmsnorm(b, b, a, 0, 32, 1e-5),
                 lambda s: s.swiglu(a, b, 32), lambda s: s.residual_add(b, a, 32)):
        with pytest.raises(vb.HipError):
            with ctx.segment() as seg:
                call(seg)


# ---------------------------------------------------------------- model

class TinyModel:
    """n_layers decode layers, an output norm and a vocab projection, every
    tensor in one weights buffer at 32-byte aligned offsets (GGUF's default
    alignment); norm weights f32, projections GGUF blocks."""

    def __init__(self, orc, c, n_layers, vocab, kinds, seed):
        from vantablack_amd.layer import LayerOffsets
        rng = np.random.default_rng(seed)
        parts, pos = [], 0

        def put(arr):
            nonlocal pos
            b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
            off = pos
            parts.append(b)
            pos += b.size
            pad = (-pos) % 32
            if pad:
                parts.append(np.zeros(pad, np.uint8))
                pos += pad
            return off

        kv_dim = c.n_kv_heads * c.head_dim
        shapes = {"q": (c.dim, c.dim), "k": (kv_dim, c.dim), "v": (kv_dim, c.dim), "o": (c.dim, c.dim),
                  "gate": (c.ffn_dim, c.dim), "up": (c.ffn_dim, c.dim), "down": (c.dim, c.ffn_dim)}
        self.offsets, self.oracle_layers = [], []
        for l in range(n_layers):
            an = (1 + 0.1 * rng.standard_normal(c.dim)).astype(np.float32)
            fn = (1 + 0.1 * rng.standard_normal(c.dim)).astype(np.float32)
            w = {n: random_weights(kinds[n], m, k, seed=seed * 100 + 10 * l + i)
                 for i, (n, (m, k)) in enumerate(shapes.items())}
            o = {n: put(w[n]) for n in shapes}
            self.offsets.append(LayerOffsets(put(an), o["q"], o["k"], o["v"], o["o"], put(fn), o["gate"], o["up"],
                                             o["down"], kinds["q"], kinds["k"], kinds["v"], kinds["o"],
                                             kinds["gate"], kinds["up"], kinds["down"]))
            # One kind per oracle layer (its matmuls take one): the model
            # uses one kind per layer for the oracle's sake.
            assert len({kinds[n] for n in shapes}) == 1
            self.oracle_layers.append(orc.LayerWeights(kinds["q"], an, w["q"], w["k"], w["v"], w["o"], fn,
                                                       w["gate"], w["up"], w["down"]))
        self.out_norm = (1 + 0.1 * rng.standard_normal(c.dim)).astype(np.float32)
        self.out_norm_off = put(self.out_norm)
        self.out_kind = kinds["out"]
        self.w_out = random_weights(self.out_kind, vocab, c.dim, seed=seed + 7)
        self.out_off = put(self.w_out)
        self.blob = np.concatenate(parts)


@pytest.mark.parametrize("path", ["layer_steps", "token_step"])
@pytest.mark.parametrize("variant", ["llama_q4_k", "gemma_like_q6_k_window", "mistral_q8_0_gqa_window"])
def test_model_decode_matches_cpu_layer_steps(ctx, orc, variant, path):
    """path layer_steps: gpu_layer_step per layer + gpu_final_step (the
    reference's encoder sequence); token_step: gpu_token_step (residual adds
    fused into the following rmsnorm)."""
    import vantablack_amd as vb
    from vantablack_amd.layer import LayerConfig, LayerScratch, gpu_final_step, gpu_layer_step, gpu_token_step
    if variant == "llama_q4_k":
        c = LayerConfig(dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn_dim=512, max_seq=16, kv_dtype=vb.F32)
        kind, n_tok = "q4_k", 5
    elif variant == "gemma_like_q6_k_window":
        c = LayerConfig(dim=512, n_heads=2, n_kv_heads=1, head_dim=256, ffn_dim=768, max_seq=16, rms_eps=1e-6,
                        rope_half=True, activation="gelu_approx", sliding_window=3, kv_dtype=vb.F32)
        kind, n_tok = "q6_k", 6
    else:
        c = LayerConfig(dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768, max_seq=16,
                        sliding_window=4, kv_dtype=vb.F32)
        kind, n_tok = "q8_0", 7
    n_layers, vocab = 2, 777 if kind != "q4_k" else 768
    kinds = {n: kind for n in ("q", "k", "v", "o", "gate", "up", "down")}
    kinds["out"] = "q8_0"
    m = TinyModel(orc, c, n_layers, vocab, kinds, seed=len(variant))
    wbuf = ctx.to_device(m.blob)
    kv_bytes = n_layers * c.max_seq * c.n_kv_heads * c.head_dim * 4
    kk, kvv = ctx.alloc(kv_bytes), ctx.alloc(kv_bytes)
    s = LayerScratch(ctx, c, vocab)
    cache = orc.OracleKvCache(n_layers, c.n_kv_heads, c.head_dim, c.max_seq)
    oc = orc.config(c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq, c.sliding_window)
    rng = np.random.default_rng(11)
    try:
        for pos in range(n_tok):
            x = rng.standard_normal(c.dim).astype(np.float32)
            ctx.upload(s.x, x)
            with ctx.segment() as seg:
                if path == "token_step":
                    gpu_token_step(seg, s, wbuf, m.offsets, kk, kvv, c, pos, m.out_norm_off, m.out_off, m.out_kind,
                                   vocab)
                else:
                    for l in range(n_layers):
                        gpu_layer_step(seg, s, wbuf, m.offsets[l], kk, kvv, c, l, pos)
                    gpu_final_step(seg, s, wbuf, m.out_norm_off, m.out_off, m.out_kind, c, vocab)
            ctx.wait_idle()
            got_x = ctx.download(s.x, np.float32, c.dim)
            got_logits = ctx.download(s.logits, np.float32, vocab)

            cache.pos = pos
            xr = x
            for l in range(n_layers):
                xr = orc.cpu_layer_step(xr, m.oracle_layers[l], cache, oc, l, c.dim, c.ffn_dim, c.rms_eps,
                                        c.rope_base, c.rope_half, c.activation)
            xr = orc.rms_norm(xr, m.out_norm, c.rms_eps)
            logits = orc.matmul_quant(m.out_kind, m.w_out, xr, vocab, c.dim)

            assert np.max(np.abs(got_x - xr)) <= 1e-4 * np.max(np.abs(xr)), f"{variant} pos {pos}: x"
            bar = 1e-4 * np.max(np.abs(logits))
            assert np.max(np.abs(got_logits - logits)) <= bar, f"{variant} pos {pos}: logits"
            top2 = np.sort(logits)[-2:]
            if top2[1] - top2[0] > bar:
                assert orc.argmax(got_logits) == orc.argmax(logits), f"{variant} pos {pos}: argmax"
    finally:
        s.release()
        for b in (wbuf, kk, kvv):
            b.release()


@pytest.mark.parametrize("kv", ["f16", "bf16"])
@pytest.mark.parametrize("variant", ["llama_q4_k", "mistral_q8_0_gqa_window"])
def test_model_decode_half_cache(ctx, orc, variant, kv):
    """gpu_token_step (grouped GEMVs, fused RoPE + append + attention, fused
    residual + rmsnorm) over an f16 / bf16 cache -- the bench's full_decode
    configuration -- against cpu_layer_step with the stored K/V rows rounded
    to the cache dtype (queries stay f32).  The decode attention computes in
    f32 on the rounded rows, so the f32 bar holds: 1e-4 of the largest value."""
    import vantablack_amd as vb
    from vantablack_amd.layer import LayerConfig, LayerScratch, gpu_token_step
    dt = vb.F16 if kv == "f16" else vb.BF16
    if variant == "llama_q4_k":
        c = LayerConfig(dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn_dim=512, max_seq=16, kv_dtype=dt)
        kind, n_tok = "q4_k", 6
    else:
        c = LayerConfig(dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768, max_seq=16,
                        sliding_window=4, kv_dtype=dt)
        kind, n_tok = "q8_0", 8
    rnd = _f16_round if kv == "f16" else _bf16_round
    n_layers, vocab = 2, 768
    kinds = dict({n: kind for n in ("q", "k", "v", "o", "gate", "up", "down")}, out="q8_0")
    m = TinyModel(orc, c, n_layers, vocab, kinds, seed=len(variant) + 3)
    wbuf = ctx.to_device(m.blob)
    kv_bytes = n_layers * c.max_seq * c.n_kv_heads * c.head_dim * 2
    kk, kvv = ctx.alloc(kv_bytes), ctx.alloc(kv_bytes)
    s = LayerScratch(ctx, c, vocab)
    cache = orc.OracleKvCache(n_layers, c.n_kv_heads, c.head_dim, c.max_seq)
    oc = orc.config(c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq, c.sliding_window)
    rng = np.random.default_rng(12)
    try:
        for pos in range(n_tok):
            x = rng.standard_normal(c.dim).astype(np.float32)
            ctx.upload(s.x, x)
            with ctx.segment() as seg:
                gpu_token_step(seg, s, wbuf, m.offsets, kk, kvv, c, pos, m.out_norm_off, m.out_off, m.out_kind, vocab)
            ctx.wait_idle()
            got_x = ctx.download(s.x, np.float32, c.dim)
            got_logits = ctx.download(s.logits, np.float32, vocab)
            cache.pos = pos
            xr = x
            for l in range(n_layers):
                xr = orc.cpu_layer_step(xr, m.oracle_layers[l], cache, oc, l, c.dim, c.ffn_dim, c.rms_eps,
                                        c.rope_base, c.rope_half, c.activation, kv_round=rnd)
            xr = orc.rms_norm(xr, m.out_norm, c.rms_eps)
            logits = orc.matmul_quant(m.out_kind, m.w_out, xr, vocab, c.dim)
            assert np.max(np.abs(got_x - xr)) <= 1e-4 * np.max(np.abs(xr)), f"{variant} {kv} pos {pos}: x"
            bar = 1e-4 * np.max(np.abs(logits))
            assert np.max(np.abs(got_logits - logits)) <= bar, f"{variant} {kv} pos {pos}: logits"
            top2 = np.sort(logits)[-2:]
            if top2[1] - top2[0] > bar:
                assert orc.argmax(got_logits) == orc.argmax(logits), f"{variant} {kv} pos {pos}: argmax"
        # The appended rows are the cache-dtype rounding of K rows that agree
        # with the oracle's to f32 summation order: at most one step of the
        # cache dtype apart.
        step = 2.0 ** -10 if kv == "f16" else 2.0 ** -7
        for l in range(n_layers):
            bits = ctx.download(kk, np.uint16, n_tok * c.n_kv_heads * c.head_dim,
                                offset=l * c.max_seq * c.n_kv_heads * c.head_dim * 2)
            got_k = orc.f16_bits_to_f32(bits) if kv == "f16" else orc.bf16_bits_to_f32(bits)
            ref_k = cache.layer_rows("k", l)[:n_tok].reshape(-1)
            assert np.all(np.abs(got_k - ref_k) <= step * np.abs(ref_k) + 1e-30), f"{variant} {kv}: layer {l} K rows"
    finally:
        s.release()
        for b in (wbuf, kk, kvv):
            b.release()


# ---------------------------------------------------------------- prefill

@pytest.mark.parametrize("n", [4096, 1003])
def test_rmsnorm_rows(ctx, orc, n):
    rows = 5
    rng = np.random.default_rng(n + 3)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    xb, wb, ob = ctx.to_device(x), ctx.to_device(w), ctx.alloc(rows * n * 4)
    with ctx.segment() as seg:
        seg.rmsnorm_rows(ob, xb, wb, 0, n, rows, 1e-5)
    got = ctx.download(ob, np.float32, rows * n).reshape(rows, n)
    for r in range(rows):
        ref = orc.rms_norm(x[r], w, 1e-5)
        assert np.max(np.abs(got[r] - ref)) <= 2e-6 * np.max(np.abs(ref)), f"row {r}"


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("heads,hd,pos0", [(8, 128, 0), (3, 256, 70000), (5, 64, 12)])
def test_rope_rows(ctx, orc, heads, hd, pos0, half):
    # Bar: 2e-6 of each head's largest value, as the decode path's fused RoPE
    # is held to the oracle's math.rope / ropeHalf.
    rows = 9
    rng = np.random.default_rng(hd + heads)
    x = rng.standard_normal((rows, heads, hd)).astype(np.float32)
    xb = ctx.to_device(x)
    with ctx.segment() as seg:
        seg.rope_rows(xb, rows, heads, hd, pos0, 10000.0, half)
    got = ctx.download(xb, np.float32, x.size).reshape(rows, heads, hd)
    for t in range(rows):
        ref = orc.rope(x[t], pos0 + t, 10000.0, half)
        assert np.all(np.max(np.abs(got[t] - ref), axis=1) <= 2e-6 * np.max(np.abs(ref), axis=1)), f"row {t}"


def _bf16_round(a):
    from oracle import oracle as o
    return o.bf16_bits_to_f32(o.f32_to_bf16_bits(np.ascontiguousarray(a, np.float32))).reshape(a.shape)


def _f16_round(a):
    from oracle import oracle as o
    return o.f16_bits_to_f32(o.f32_to_f16_bits(np.ascontiguousarray(a, np.float32))).reshape(a.shape)


@pytest.mark.parametrize("variant", ["llama_q4_k_f32cache", "mistral_q8_0_bf16_window_pos7"])
def test_model_prefill_matches_cpu_prefill_layers(ctx, orc, variant):
    """Two layers of prefill on the GPU (gpu_prefill_layer: MFMA projections
    and attention, batched RoPE, per-token norms) against
    oracle.cpu_prefill_layer (prefillLayer, prefill.zig:151-231).  Bars: 1e-4 of
    the residual stream's largest value with an f32 cache; 2e-3 with a bf16
    cache (keys and values rounded to bf16 on both sides, queries f32 on
    both; f16 MFMA operands, two-piece where this model's large scores call
    for it)."""
    import vantablack_amd as vb
    from vantablack_amd.layer import LayerConfig, PrefillScratch, gpu_prefill_layer
    if variant == "llama_q4_k_f32cache":
        c = LayerConfig(dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn_dim=512, max_seq=64, kv_dtype=vb.F32)
        kind, B, pos0, bar, rnd = "q4_k", 37, 0, 1e-4, None
    else:
        c = LayerConfig(dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768, max_seq=80, sliding_window=20,
                        kv_dtype=vb.BF16)
        kind, B, pos0, bar, rnd = "q8_0", 50, 7, 2e-3, _bf16_round
    n_layers = 2
    kinds = dict({n: kind for n in ("q", "k", "v", "o", "gate", "up", "down")}, out="q8_0")
    m = TinyModel(orc, c, n_layers, 64, kinds, seed=len(variant))
    wbuf = ctx.to_device(m.blob)
    kv_dim = c.n_kv_heads * c.head_dim
    rng = np.random.default_rng(23)
    cache = orc.OracleKvCache(n_layers, c.n_kv_heads, c.head_dim, c.max_seq)
    # Rows before pos0 (an earlier prompt): random, in the cache's precision.
    prior_k = rng.standard_normal((n_layers, pos0, kv_dim)).astype(np.float32)
    prior_v = rng.standard_normal((n_layers, pos0, kv_dim)).astype(np.float32)
    if rnd is not None:
        prior_k, prior_v = rnd(prior_k), rnd(prior_v)
    for l in range(n_layers):
        cache.layer_rows("k", l)[:pos0] = prior_k[l].reshape(pos0, c.n_kv_heads, c.head_dim)
        cache.layer_rows("v", l)[:pos0] = prior_v[l].reshape(pos0, c.n_kv_heads, c.head_dim)
    if c.kv_dtype == vb.F32:
        kfull = np.zeros((n_layers, c.max_seq, kv_dim), np.float32)
        vfull = np.zeros_like(kfull)
    else:
        kfull = np.zeros((n_layers, c.max_seq, kv_dim), np.uint16)
        vfull = np.zeros_like(kfull)
    kfull[:, :pos0] = prior_k if c.kv_dtype == vb.F32 else orc.f32_to_bf16_bits(prior_k).reshape(prior_k.shape)
    vfull[:, :pos0] = prior_v if c.kv_dtype == vb.F32 else orc.f32_to_bf16_bits(prior_v).reshape(prior_v.shape)
    kk, kvv = ctx.to_device(kfull), ctx.to_device(vfull)
    s = PrefillScratch(ctx, c, B)
    x = rng.standard_normal((B, c.dim)).astype(np.float32)
    oc = orc.config(c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq, c.sliding_window)
    try:
        ctx.upload(s.x, x)
        with ctx.segment() as seg:
            for l in range(n_layers):
                gpu_prefill_layer(seg, s, wbuf, m.offsets[l], kk, kvv, c, l, pos0)
        ctx.wait_idle()
        got = ctx.download(s.x, np.float32, B * c.dim).reshape(B, c.dim)
        cache.pos = pos0
        xr = x
        for l in range(n_layers):
            xr = orc.cpu_prefill_layer(xr, m.oracle_layers[l], cache, oc, l, c.dim, c.ffn_dim, c.rms_eps,
                                       c.rope_base, c.rope_half, c.activation, kv_round=rnd)
        assert np.max(np.abs(got - xr)) <= bar * np.max(np.abs(xr)), f"{variant}: max err " \
            f"{np.max(np.abs(got - xr)) / np.max(np.abs(xr)):.2e}"
    finally:
        s.release()
        for b in (wbuf, kk, kvv):
            b.release()


def test_new_entries_reject_bad_shapes_and_ranges(ctx):
    """Bad arguments to the batched and grouped entries are recorded on the
    segment and reported by commit, never launched."""
    import vantablack_amd as vb
    from vantablack_amd import hip
    small, big = ctx.alloc(256), ctx.alloc(1 << 20)
    calls = [
        lambda s: s.rmsnorm_rows(big, small, big, 0, 64, 4, 1e-5),        # rows beyond the input
        lambda s: s.rope_rows(big, 2, 4, 63, 0, 10000.0),                 # odd head_dim
        lambda s: s.rope_rows(small, 4, 4, 64, 0, 10000.0),               # rows beyond the buffer
        lambda s: s.matmul3("q8_0", small, big, 64, [(big, 0, 64), (big, 0, 64)]),   # weights beyond the buffer
        lambda s: s.matmul_gated("q4_k", big, big, 0, 0, big, 64, 100),   # k not a whole number of blocks
        lambda s: hip.lib().vtb_hip_segment_matmul_gated_q8_0(s.h, big.h, big.h, 0, 0, big.h, 8, 64, 7),  # activation
    ]
    for i, call in enumerate(calls):
        with pytest.raises(vb.HipError):
            with ctx.segment() as seg:
                call(seg)
