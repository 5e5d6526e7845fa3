"""XCD-local split merge on the GPU: with the workgroups of a unit on one XCD
(vtb_hip_xcd_map > 0) the split partials travel through that XCD's L2.  The
arithmetic and its order are those of the agent-coherent merge, so the
outputs must be bit-identical to a context with VTB_DECODE_XCD_LOCAL=0, and
within the north-star tolerance of the oracle (forward.zig:187-228)."""
import os

import numpy as np
import pytest

from tests.parity import check, make_kv

pytestmark = pytest.mark.gpu


def _ctx(xcl):
    import vantablack_amd as vb
    old = os.environ.get("VTB_DECODE_XCD_LOCAL")
    os.environ["VTB_DECODE_XCD_LOCAL"] = "1" if xcl else "0"
    try:
        return vb.Context()
    finally:
        if old is None:
            del os.environ["VTB_DECODE_XCD_LOCAL"]
        else:
            os.environ["VTB_DECODE_XCD_LOCAL"] = old


@pytest.fixture(scope="module")
def ctxs():
    on, off = _ctx(True), _ctx(False)
    yield on, off
    on.close()
    off.close()


def _run(ctx, n_heads, n_kv, d, pos, dtype, window, ks, vs, q, kx, vx, steps):
    """`steps` decode steps from pos through vtb_hip_layer_attention (slot
    write + attention); returns every step's output."""
    import vantablack_amd as vb
    max_seq = pos + steps
    W = vb.NO_WINDOW if window is None else window
    cache = vb.KvCache(ctx, 1, n_kv, d, max_seq, dtype)
    outs = []
    try:
        cache.write_rows("k", 0, 0, ks[:pos])
        cache.write_rows("v", 0, 0, vs[:pos])
        cache.pos = pos
        c = vb.LlamaConfig(n_heads, n_kv, d, max_seq, W)
        qb, ob = ctx.to_device(q), ctx.alloc(n_heads * d * 4)
        for s in range(steps):
            kb, vb_ = ctx.to_device(kx[pos + s].reshape(-1)), ctx.to_device(vx[pos + s].reshape(-1))
            with ctx.segment() as seg:
                vb.layer_attention(seg, cache, c, 0, qb, kb, vb_, ob)
            ctx.wait_idle()
            outs.append(ctx.download(ob, np.float32, n_heads * d))
            cache.pos = pos + s + 1
    finally:
        cache.close()
    return outs


# (n_heads, n_kv, d, pos, dtype, window): the MFMA form takes the XCD-local
# merge when its units divide over the XCDs -- C3's shape (GQA 4:1 bf16,
# window 4096 at 16383, 8 units), groups of 4, 8 and 16 at other lengths and
# head_dims; C2's shape (scalar head-group form) and an f32 cache keep the
# coherent merge in both contexts and are compared all the same.
CASES = [
    (32, 8, 128, 16383, "bf16", 4096),
    (32, 8, 128, 3000, "bf16", None),
    (64, 16, 64, 5000, "f16", None),
    (64, 8, 128, 4000, "bf16", None),
    (128, 8, 128, 2000, "f16", None),
    (32, 32, 128, 8192, "f16", None),
    (16, 16, 128, 777, "f32", None),
]


@pytest.mark.parametrize("n_heads,n_kv,d,pos,dtype,window", CASES)
def test_xcd_local_merge_is_bit_identical(ctxs, orc, n_heads, n_kv, d, pos, dtype, window):
    on, off = ctxs
    if on.xcd_map == 0:
        pytest.skip("workgroups are not dealt round-robin over XCDs on this device: XCD-local merge off")
    assert off.xcd_map == 0
    steps = 3
    ks, kx, vs, vx = make_kv(orc, pos + steps, n_kv, d, dtype, seed=pos % 97)
    q = orc.normal(pos + 11, n_heads * d)
    got_on = _run(on, n_heads, n_kv, d, pos, dtype, window, ks, vs, q, kx, vx, steps)
    got_off = _run(off, n_heads, n_kv, d, pos, dtype, window, ks, vs, q, kx, vx, steps)
    for s in range(steps):
        assert np.array_equal(got_on[s], got_off[s]), f"step {s}: XCD-local merge differs from the coherent merge"
    # The last step against the oracle.
    W = orc.NO_WINDOW if window is None else window
    p = pos + steps - 1
    ocache = orc.OracleKvCache(1, n_kv, d, p + 1)
    ocache.layer_rows("k", 0)[:p + 1] = kx[:p + 1]
    ocache.layer_rows("v", 0)[:p + 1] = vx[:p + 1]
    ocache.pos = p
    ref = orc.cpu_attention(q, ocache, orc.config(n_heads, n_kv, d, p + 1, W), 0)
    check(orc, got_on[-1], ref, n_heads, dtype, what=f"xcd-local decode h{n_heads}/{n_kv} d{d} pos{p} {dtype}")


def test_xcd_map_reported(ctxs):
    on, off = ctxs
    print(f"xcd_map: {on.xcd_map} (off context {off.xcd_map})", flush=True)
    assert off.xcd_map == 0
    assert on.xcd_map in (0, 1, 2, 4, 8)
