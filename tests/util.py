"""Shared helpers for the parity tests (CPU side)."""
import numpy as np


def rel_err(got, ref, n_rows) -> float:
    """Parity metric used throughout: for every head (row of the output),
    max_i |got_i - ref_i| / max_i |ref_i|, then the max over heads.  An
    element-wise relative error is meaningless where the reference output is
    ~0, so the normaliser is the row's largest magnitude."""
    g = np.asarray(got, np.float64).reshape(n_rows, -1)
    r = np.asarray(ref, np.float64).reshape(n_rows, -1)
    den = np.max(np.abs(r), axis=1)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(np.max(np.abs(g - r), axis=1) / den))


def np_attention_f64(q, K, V, n_heads, n_kv, d, cur_pos, window, kv_map=None, scale=None):
    """Independent vectorised formula: softmax(q K^T * scale) V in f64 over
    rows [window_start, cur_pos].  K, V: [rows, n_kv, d] (one layer)."""
    q = np.asarray(q, np.float64).reshape(n_heads, d)
    ws = 0 if (window is None or cur_pos < window) else cur_pos - window + 1
    sc = (1.0 / np.sqrt(d)) if scale is None else scale
    out = np.zeros((n_heads, d))
    for h in range(n_heads):
        kvh = (h * n_kv) // n_heads if kv_map is None else kv_map(h)
        k = np.asarray(K[ws:cur_pos + 1, kvh], np.float64)
        v = np.asarray(V[ws:cur_pos + 1, kvh], np.float64)
        s = (k @ q[h]) * sc
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out.reshape(-1)


def fill_cache_random(orc, cache, n_rows, seed):
    """Fill rows [0, n_rows) of every layer's K and V with seeded normals."""
    L = cache.c.n_layers
    row = cache.row
    for layer in range(L):
        for which, s in (("k", 2 * seed + 1), ("v", 2 * seed + 2)):
            vals = orc.normal(s * 1000 + layer, n_rows * row).reshape(n_rows, cache.c.n_kv_heads, cache.c.head_dim)
            cache.layer_rows(which, layer)[:n_rows] = vals
