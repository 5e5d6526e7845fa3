"""Writes the committed golden vectors (run from the repo root):
    python tests/golden/make_golden.py

Inputs are regenerated from the seeded portable RNG (oracle/oracle.py); the
fixtures hold the oracle's outputs plus a SHA-256 of the inputs, so a later
change to the RNG, the oracle or the input recipe is caught by
tests/test_golden.py before any GPU comparison is trusted.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402


def sha(*arrs):
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def c1_inputs():
    n_heads, n_kv, d, L = 32, 4, 64, 512
    s = np.float32(1.0 / np.sqrt(d))
    k = (orc.normal(0, L * n_kv * d, offset=0) * s).reshape(L, n_kv, d)
    v = (orc.normal(0, L * n_kv * d, offset=L * n_kv * d) * s).reshape(L, n_kv, d)
    q = orc.normal(0, n_heads * d, offset=2 * L * n_kv * d) * s
    return q, k, v


def c1_output(q, k, v):
    oc = orc.OracleKvCache(1, 4, 64, 512)
    oc.layer_rows("k", 0)[:] = k
    oc.layer_rows("v", 0)[:] = v
    oc.pos = 511
    return orc.cpu_attention(q, oc, orc.config(32, 4, 64, 512), 0)


# Tiny cases: (name, n_heads, n_kv, d, dtype, n_rows, pos0, n_tokens, window, seed)
TINY = [
    ("gqa4_f16_decode", 8, 2, 64, "f16", 100, 99, 1, None, 11),
    ("mqa_d256_bf16_decode", 8, 1, 256, "bf16", 70, 69, 1, None, 12),
    ("swa_bf16_decode", 4, 2, 128, "bf16", 90, 89, 1, 32, 13),
    ("causal_prefill_bf16", 4, 2, 128, "bf16", 48, 0, 48, None, 14),
    ("causal_prefill_swa_f16", 4, 4, 64, "f16", 80, 16, 64, 24, 15),
]


def tiny_inputs(n_heads, n_kv, d, dtype, n_rows, n_tokens, seed):
    """Seeded inputs of a tiny case: (q, q, k stored, k exact, v stored,
    v exact).  The queries are f32 for every cache dtype, as the reference's
    State.q / s.q are (forward.zig:37, prefill.zig:167-197); only the cache
    rows take the cache dtype.  q is returned twice so callers can unpack the
    stored/exact pairs uniformly."""
    k = orc.normal(seed * 10 + 1, n_rows * n_kv * d).reshape(n_rows, n_kv, d)
    v = orc.normal(seed * 10 + 2, n_rows * n_kv * d).reshape(n_rows, n_kv, d)
    q = orc.normal(seed * 10 + 3, n_tokens * n_heads * d).reshape(n_tokens, n_heads * d)
    ks, kx = orc.to_dtype(k, dtype)
    vs, vx = orc.to_dtype(v, dtype)
    return (q, q, ks.reshape(k.shape), kx.reshape(k.shape), vs.reshape(v.shape), vx.reshape(v.shape))


def tiny_output(case):
    name, n_heads, n_kv, d, dtype, n_rows, pos0, n_tok, window, seed = case
    qs, qx, ks, kx, vs, vx = tiny_inputs(n_heads, n_kv, d, dtype, n_rows, n_tok, seed)
    W = orc.NO_WINDOW if window is None else window
    oc = orc.OracleKvCache(1, n_kv, d, n_rows)
    oc.layer_rows("k", 0)[:] = kx
    oc.layer_rows("v", 0)[:] = vx
    oc.pos = pos0
    out = orc.attention_causal(qx.reshape(-1), oc, orc.config(n_heads, n_kv, d, n_rows, W), 0, range(n_tok))
    return out, (qs, ks, vs)


def main():
    q, k, v = c1_inputs()
    out = c1_output(q, k, v)
    np.savez(os.path.join(HERE, "c1_decode.npz"), out=out, inputs_sha256=np.array(sha(q, k, v)))
    for case in TINY:
        out, ins = tiny_output(case)
        np.savez(os.path.join(HERE, f"{case[0]}.npz"), out=out, inputs_sha256=np.array(sha(*ins)))
    print("wrote", 1 + len(TINY), "fixtures")


if __name__ == "__main__":
    main()
