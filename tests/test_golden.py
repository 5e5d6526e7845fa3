"""Golden vectors: the oracle reproduces its committed fixtures bit-exactly
from the seeded inputs (CPU), and the HIP path matches them (GPU)."""
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg
from tests.parity import check

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, f"{name}.npz"))


def test_c1_fixture_reproduces(orc):
    q, k, v = mg.c1_inputs()
    f = load("c1_decode")
    assert str(f["inputs_sha256"]) == mg.sha(q, k, v)
    assert np.array_equal(mg.c1_output(q, k, v), f["out"])


@pytest.mark.parametrize("case", mg.TINY, ids=[c[0] for c in mg.TINY])
def test_tiny_fixture_reproduces(orc, case):
    out, ins = mg.tiny_output(case)
    f = load(case[0])
    assert str(f["inputs_sha256"]) == mg.sha(*ins)
    assert np.array_equal(out, f["out"])


DECODE_CASES = [c for c in mg.TINY if c[7] == 1]


@pytest.mark.gpu
@pytest.mark.parametrize("case", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_tiny_decode_fixture_on_gpu(ctx, orc, case):
    import vantablack_amd as vb
    name, n_heads, n_kv, d, dtype, n_rows, pos0, n_tok, window, seed = case
    qs, qx, ks, kx, vs, vx = mg.tiny_inputs(n_heads, n_kv, d, dtype, n_rows, n_tok, seed)
    ws = orc.window_start(pos0, orc.NO_WINDOW if window is None else window)
    L = pos0 + 1 - ws
    rb = n_kv * d * (4 if dtype == "f32" else 2)
    kb, vbuf, qb, ob = ctx.to_device(ks), ctx.to_device(vs), ctx.to_device(qx), ctx.alloc(n_heads * d * 4)
    with ctx.segment() as seg:
        seg.attn_decode(ob, qb, kb, ws * rb, vbuf, ws * rb, n_heads, n_kv, d, L, 1.0 / np.sqrt(d),
                        vb.hip.DTYPES[dtype])
    got = ctx.download(ob, np.float32, n_heads * d)
    check(orc, got, load(name)["out"], n_heads, dtype, what=name)
