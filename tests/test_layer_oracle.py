"""CPU checks of the decode-layer restatements in oracle/attn_oracle.c --
math.rmsNorm (src/kernels/math.zig:11-32), math.swiglu (:154-161) and
math.gegluApprox (:166-175) -- and of oracle.cpu_layer_step (forward.zig:
230-288), against what the mathematics fixes: closed forms, odd symmetries,
an independent f64 formula, and a planted mistake that must be caught."""
import numpy as np
import pytest

from tests.quant import np_dequant, random_weights


def test_rmsnorm_constant_row_closed_form(orc):
    for n, c, eps in [(8, 3.0, 1e-5), (37, -0.5, 1e-6), (4096, 2.0, 1e-5)]:
        x = np.full(n, c, np.float32)
        w = np.linspace(0.5, 1.5, n).astype(np.float32)
        got = orc.rms_norm(x, w, eps)
        ref = w.astype(np.float64) * c / np.sqrt(c * c + eps)
        assert np.allclose(got, ref, rtol=2e-6, atol=0)


@pytest.mark.parametrize("n", [1, 7, 8, 4095, 5000])
def test_rmsnorm_f64_formula_and_scale_invariance(orc, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd * w / np.sqrt(np.mean(xd * xd) + 1e-5)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))
    # eps = 0: scaling x by a power of two changes nothing, bit for bit.
    assert np.array_equal(orc.rms_norm(x, w, 0.0), orc.rms_norm(x * np.float32(8.0), w, 0.0))


def test_rmsnorm_closed_form_catches_a_wrong_mean():
    # A restatement that averaged over n - 1 would miss the closed form by
    # far more than the 2e-6 bar above.
    n, c, eps = 16, 2.0, 1e-5
    right = c / np.sqrt(c * c + eps)
    wrong = c / np.sqrt(c * c * n / (n - 1) + eps)
    assert abs(right - wrong) > 1e-2


def test_swiglu_closed_forms_and_symmetry(orc):
    z = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 3.5], np.float32)
    s = orc.swiglu(z, np.ones_like(z))
    zd = z.astype(np.float64)
    assert s[0] == 0.0
    assert np.allclose(s, zd / (1 + np.exp(-zd)), rtol=2e-7, atol=1e-12)
    rng = np.random.default_rng(2)
    z = (rng.standard_normal(1000) * 4).astype(np.float32)
    one = np.ones_like(z)
    # silu(z) - silu(-z) = z (the sigmoid's odd part); a sign slip in exp(-z) fails this
    d = orc.swiglu(z, one).astype(np.float64) - orc.swiglu(-z, one).astype(np.float64)
    assert np.max(np.abs(d - z)) <= 4e-6 * np.max(np.abs(z))
    u = rng.standard_normal(1000).astype(np.float32)
    assert np.array_equal(orc.swiglu(z, u), orc.swiglu(z, one) * u)


def test_gelu_approx_closed_forms_and_symmetry(orc):
    z = np.array([0.0, 1.0, -1.0, 6.0, -6.0], np.float32)
    g = orc.geglu_approx(z, np.ones_like(z))
    zd = z.astype(np.float64)
    ref = 0.5 * zd * (1 + np.tanh(np.sqrt(2 / np.pi) * (zd + 0.044715 * zd ** 3)))
    assert g[0] == 0.0
    assert np.allclose(g, ref, rtol=2e-6, atol=1e-7)
    rng = np.random.default_rng(3)
    z = (rng.standard_normal(1000) * 3).astype(np.float32)
    one = np.ones_like(z)
    # gelu(z) - gelu(-z) = z (tanh is odd)
    d = orc.geglu_approx(z, one).astype(np.float64) - orc.geglu_approx(-z, one).astype(np.float64)
    assert np.max(np.abs(d - z)) <= 4e-6 * np.max(np.abs(z))


def _rope_f64(x, pos, base, half):
    d = x.shape[-1]
    j = np.arange(d // 2)
    th = pos / np.power(float(base), 2.0 * j / d)
    c, s = np.cos(th), np.sin(th)
    y = x.copy()
    if half:
        a, b = x[..., : d // 2], x[..., d // 2:]
        y[..., : d // 2], y[..., d // 2:] = a * c - b * s, a * s + b * c
    else:
        a, b = x[..., 0::2], x[..., 1::2]
        y[..., 0::2], y[..., 1::2] = a * c - b * s, a * s + b * c
    return y


@pytest.mark.parametrize("activation,half", [("silu", False), ("gelu_approx", True)])
def test_cpu_layer_step_matches_an_f64_layer(orc, activation, half):
    """Three tokens through one layer: the composition (norm, projections,
    RoPE, cache write, attention, residuals, gated FFN) against the same
    layer written out in f64 with dequantised weights."""
    dim, nh, nkv, hd, ffn, kind = 64, 2, 1, 32, 128, "q8_0"
    rng = np.random.default_rng(7)
    ws = {n: random_weights(kind, m, k, seed=s) for s, (n, m, k) in enumerate(
        [("q", dim, dim), ("k", nkv * hd, dim), ("v", nkv * hd, dim), ("o", dim, dim),
         ("gate", ffn, dim), ("up", ffn, dim), ("down", dim, ffn)])}
    an = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    fn = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    lw = orc.LayerWeights(kind, an, ws["q"], ws["k"], ws["v"], ws["o"], fn, ws["gate"], ws["up"], ws["down"])
    W = {n: np_dequant(kind, w).astype(np.float64).reshape(-1, k)
         for (n, w), k in zip(ws.items(), [dim] * 6 + [ffn])}
    cache = orc.OracleKvCache(1, nkv, hd, 8)
    c = orc.config(nh, nkv, hd, 8)
    keys, vals = [], []
    for pos in range(3):
        x = rng.standard_normal(dim).astype(np.float32)
        cache.pos = pos
        got = orc.cpu_layer_step(x, lw, cache, c, 0, dim, ffn, 1e-5, 10000.0, half, activation)
        xd = x.astype(np.float64)
        h = xd * an / np.sqrt(np.mean(xd * xd) + 1e-5)
        q = _rope_f64((W["q"] @ h).reshape(nh, hd), pos, 10000.0, half)
        keys.append(_rope_f64((W["k"] @ h).reshape(nkv, hd), pos, 10000.0, half))
        vals.append((W["v"] @ h).reshape(nkv, hd))
        K, V = np.stack(keys), np.stack(vals)
        att = np.zeros((nh, hd))
        for hh in range(nh):
            kv = hh * nkv // nh
            s = K[:, kv] @ q[hh] / np.sqrt(hd)
            p = np.exp(s - s.max())
            att[hh] = (p / p.sum()) @ V[:, kv]
        xd = xd + W["o"] @ att.reshape(-1)
        h = xd * fn / np.sqrt(np.mean(xd * xd) + 1e-5)
        g, u = W["gate"] @ h, W["up"] @ h
        if activation == "silu":
            a = g / (1 + np.exp(-g)) * u
        else:
            a = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u
        ref = xd + W["down"] @ a
        assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(ref)), f"pos {pos}"


# ---- The reference's own known-answer tests (src/kernels/math.zig), ported.

def test_rmsnorm_reference_kat(orc):
    # math.zig:205-215 "rmsNorm: identity weight zeros eps": x = 1..8, w = 1,
    # eps = 0 against the f32 ss / sqrt formula, within 1e-4.
    x = np.arange(1, 9, dtype=np.float32)
    w = np.ones(8, np.float32)
    ss = np.float32(0)
    for v in x:
        ss = np.float32(ss + v * v)
    inv = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(8)))
    ref = x * inv
    got = orc.rms_norm(x, w, 0.0)
    assert np.max(np.abs(got - ref)) <= 1e-4


def test_geglu_approx_reference_kat(orc):
    # math.zig:232-241: gelu_approx at known points (the reference's own
    # high-precision values), up = 1, within 1e-4.  These pin the constants
    # sqrt(2/pi) and 0.044715, which the odd-symmetry check above cannot.
    gate = np.array([-2.0, -0.5, 0.0, 0.5, 1.0, 2.0], np.float32)
    expected = np.array([-0.045402, -0.154286, 0.0, 0.345714, 0.841192, 1.954598], np.float32)
    got = orc.geglu_approx(gate, np.ones_like(gate))
    assert np.max(np.abs(got - expected)) <= 1e-4


def test_geglu_approx_kat_catches_a_wrong_constant():
    # A restatement with 0.0447 or sqrt(1/pi) misses the known points by more
    # than the KAT's 1e-4 at z = 2.
    z = 2.0
    def g(c, k):
        return 0.5 * z * (1 + np.tanh(k * (z + c * z ** 3)))
    right = g(0.044715, np.sqrt(2 / np.pi))
    assert abs(right - 1.954598) < 1e-5
    assert abs(g(0.0447, np.sqrt(2 / np.pi)) - right) > 1e-5 or abs(g(0.044715, np.sqrt(1 / np.pi)) - right) > 1e-4
    assert abs(g(0.044715, np.sqrt(1 / np.pi)) - right) > 1e-4


def test_swiglu_reference_kat(orc):
    # math.zig:243-250 "swiglu against scalar reference": g / (1 + exp(-g)) * u
    # in f32, within 1e-5.
    g = np.array([0.5, -1.0, 2.0, 0.0], np.float32)
    u = np.array([1.0, 2.0, 0.5, 4.0], np.float32)
    ref = (g / (np.float32(1.0) + np.exp(-g))) * u
    got = orc.swiglu(g, u)
    assert np.max(np.abs(got - ref)) <= 1e-5


def test_cpu_prefill_layer_matches_an_f64_layer(orc):
    """prefillLayer restated (oracle.cpu_prefill_layer) for B tokens after an
    earlier prompt, with a sliding window, against the same layer written out
    in f64 with dequantised weights: per-token rmsnorm, batched projections,
    RoPE at pos0 + b, all B rows written before attention, causal windowed
    attention, residual, gated FFN (prefill.zig:151-231)."""
    dim, nh, nkv, ffn, kind = 256, 4, 2, 512, "q4_k"  # Q4_K blocks hold 256 weights
    hd = dim // nh
    B, pos0, W = 5, 3, 4
    rng = np.random.default_rng(17)
    ws = {n: random_weights(kind, m, k, seed=40 + s) for s, (n, m, k) in enumerate(
        [("q", dim, dim), ("k", nkv * hd, dim), ("v", nkv * hd, dim), ("o", dim, dim),
         ("gate", ffn, dim), ("up", ffn, dim), ("down", dim, ffn)])}
    an = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    fn = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    lw = orc.LayerWeights(kind, an, ws["q"], ws["k"], ws["v"], ws["o"], fn, ws["gate"], ws["up"], ws["down"])
    Wd = {n: np_dequant(kind, w).astype(np.float64).reshape(-1, k)
          for (n, w), k in zip(ws.items(), [dim] * 6 + [ffn])}
    max_seq = pos0 + B + 2
    cache = orc.OracleKvCache(1, nkv, hd, max_seq)
    prior_k = rng.standard_normal((pos0, nkv, hd)).astype(np.float32)
    prior_v = rng.standard_normal((pos0, nkv, hd)).astype(np.float32)
    cache.layer_rows("k", 0)[:pos0] = prior_k
    cache.layer_rows("v", 0)[:pos0] = prior_v
    cache.pos = pos0
    c = orc.config(nh, nkv, hd, max_seq, W)
    x = rng.standard_normal((B, dim)).astype(np.float32)
    got = orc.cpu_prefill_layer(x, lw, cache, c, 0, dim, ffn, 1e-5, 10000.0, False, "silu")
    xd = x.astype(np.float64)
    h = xd * an / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5)
    q = np.stack([_rope_f64((Wd["q"] @ h[b]).reshape(nh, hd), pos0 + b, 10000.0, False) for b in range(B)])
    k = np.stack([_rope_f64((Wd["k"] @ h[b]).reshape(nkv, hd), pos0 + b, 10000.0, False) for b in range(B)])
    v = np.stack([(Wd["v"] @ h[b]).reshape(nkv, hd) for b in range(B)])
    K = np.concatenate([prior_k.astype(np.float64), k])
    V = np.concatenate([prior_v.astype(np.float64), v])
    att = np.zeros((B, nh, hd))
    for b in range(B):
        cur = pos0 + b
        ws0 = 0 if cur < W else cur - W + 1
        for hh in range(nh):
            kv = hh * nkv // nh
            s = K[ws0:cur + 1, kv] @ q[b, hh] / np.sqrt(hd)
            p = np.exp(s - s.max())
            att[b, hh] = (p / p.sum()) @ V[ws0:cur + 1, kv]
    xd = xd + att.reshape(B, -1) @ Wd["o"].T
    h = xd * fn / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5)
    g, u = h @ Wd["gate"].T, h @ Wd["up"].T
    ref = xd + (g / (1 + np.exp(-g)) * u) @ Wd["down"].T
    assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(ref))
    # The B rows landed in the cache at pos0.. before the attention read them.
    rows = cache.layer_rows("k", 0)[pos0:pos0 + B]
    assert np.max(np.abs(rows - k)) <= 2e-5 * np.max(np.abs(k))
