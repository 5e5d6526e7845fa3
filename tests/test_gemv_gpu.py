"""Quantised GEMV on the GPU, through the C ABI, against the oracle's restatement
of src/kernels/simd.zig matmul_* (Q8_0, Q4_K, Q5_K, Q6_K).

Bars: the reference's own Metal check (bridge.zig:466-470: 1e-4 relative per
output on a random-byte fixture) and, stronger, |got - ref| <= 1e-5 *
sum_j |W_ij x_j| per row, which holds however much a row's sum cancels.
"""
import numpy as np
import pytest

from tests.quant import BLOCK, np_dequant, random_weights

pytestmark = pytest.mark.gpu
KINDS = ["q8_0", "q4_k", "q5_k", "q6_k"]


def gemv_case(ctx, orc, kind, m, k, seed, w_offset=0, x=None):
    import vantablack_amd as vb
    w = random_weights(kind, m, k, seed)
    if x is None:
        rng = np.random.default_rng(seed + 1)
        x = ((rng.random(k, dtype=np.float32) - 0.5) * 2.0).astype(np.float32)
    wbuf = ctx.to_device(np.concatenate([np.zeros(w_offset, np.uint8), w]))
    xb, ob = ctx.to_device(x), ctx.alloc(m * 4)
    with ctx.segment() as seg:
        seg.matmul_quant(kind, ob, wbuf, w_offset, xb, m, k)
    got = ctx.download(ob, np.float32, m).astype(np.float64)
    ref = orc.matmul_quant(kind, w, x, m, k).astype(np.float64)
    cond = np.abs(np_dequant(kind, w).astype(np.float64).reshape(m, k)) @ np.abs(x.astype(np.float64))
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 * cond), f"{kind} m{m} k{k}: max err/cond {np.max(err / cond):.2e}"
    big = np.abs(ref) > 1e-3 * cond
    assert np.all(err[big] <= 1e-4 * np.abs(ref[big])), f"{kind} m{m} k{k}: relative error above 1e-4"
    return got


@pytest.mark.parametrize("kind", KINDS)
def test_reference_parity_fixture(ctx, orc, kind):
    # bridge.zig:383-472: m = 4 rows, k = two blocks, random bytes with small
    # finite f16 super-scales, activations uniform in [-1, 1).
    gemv_case(ctx, orc, kind, 4, 2 * BLOCK[kind][1], seed=0xDEADBEEF % 1000 + len(kind))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m,k", [(4096, 4096), (11008, 4096), (4096, 11008)])
def test_llama2_7b_projection_shapes(ctx, orc, kind, m, k):
    gemv_case(ctx, orc, kind, m, k, seed=m + k + len(kind))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m,k", [(1, 256), (13, 2304), (1023, 512), (37, 4352)])
def test_ragged_shapes(ctx, orc, kind, m, k):
    # m not a multiple of the rows per workgroup; k ending inside a 2048-wide
    # step (2304 = 9 blocks, 4352 = 17 blocks).
    gemv_case(ctx, orc, kind, m, k, seed=m * 3 + k)


@pytest.mark.parametrize("kind", KINDS)
def test_weight_offset(ctx, orc, kind):
    gemv_case(ctx, orc, kind, 64, 1024, seed=9, w_offset=4100)


@pytest.mark.parametrize("rows", ["1", "2", "4"])
@pytest.mark.parametrize("kind", KINDS)
def test_every_rows_per_wave_variant(ctx, orc, monkeypatch, kind, rows):
    monkeypatch.setenv("VTB_GEMV_R", rows)
    gemv_case(ctx, orc, kind, 523, 2048, seed=int(rows) + 100)


def test_rejects_bad_shapes_and_alignment(ctx):
    import vantablack_amd as vb
    w = ctx.alloc(1 << 16)
    x = ctx.alloc(4096 * 4)
    o = ctx.alloc(4096 * 4)
    for kind, m, k, off in [("q4_k", 4, 300, 0),      # k not a whole number of blocks
                            ("q8_0", 4, 64, 2),       # weights not 4-byte aligned
                            ("q6_k", 400, 512, 0)]:   # weights beyond the buffer
        with pytest.raises(vb.HipError):
            with ctx.segment() as seg:
                seg.matmul_quant(kind, o, w, off, x, m, k)


def test_synchronous_entry(ctx, orc):
    import vantablack_amd as vb
    kind, m, k = "q4_k", 32, 512
    w = random_weights(kind, m, k, seed=3)
    x = orc.normal(4, k)
    wb, xb, ob = ctx.to_device(w), ctx.to_device(x), ctx.alloc(m * 4)
    assert vb.hip.lib().vtb_hip_matmul_q4_k(ctx.h, ob.h, wb.h, 0, xb.h, m, k) == 0
    got = ctx.download(ob, np.float32, m)
    ref = orc.matmul_quant(kind, w, x, m, k)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("ms", [(4096, 1024, 1024), (11008, 11008), (13, 1000, 257)])
def test_grouped_row_blocks_match_single_gemvs(ctx, orc, kind, ms):
    """vtb_hip_segment_matmul3_<kind>: two or three row blocks (their own
    weights and outputs, one activation vector) in one launch, each to the
    per-row bar of the single GEMV; block sizes not multiples of the rows per
    workgroup included."""
    k = 1024 if kind == "q8_0" else 2048
    rng = np.random.default_rng(sum(ms))
    x = ((rng.random(k, dtype=np.float32) - 0.5) * 2.0).astype(np.float32)
    ws = [random_weights(kind, m, k, seed=m + i) for i, m in enumerate(ms)]
    offs, pos = [], 0
    for w in ws:
        offs.append(pos)
        pos += (w.size + 31) // 32 * 32
    blob = np.zeros(pos, np.uint8)
    for w, o in zip(ws, offs):
        blob[o:o + w.size] = w
    wb, xb = ctx.to_device(blob), ctx.to_device(x)
    outs = [ctx.alloc(m * 4) for m in ms]
    with ctx.segment() as seg:
        seg.matmul3(kind, wb, xb, k, [(o, off, m) for o, off, m in zip(outs, offs, ms)])
    for w, o, m in zip(ws, outs, ms):
        got = ctx.download(o, np.float32, m).astype(np.float64)
        ref = orc.matmul_quant(kind, w, x, m, k).astype(np.float64)
        cond = np.abs(np_dequant(kind, w).astype(np.float64).reshape(m, k)) @ np.abs(x.astype(np.float64))
        assert np.all(np.abs(got - ref) <= 1e-5 * cond), f"{kind} block m{m}"


@pytest.mark.parametrize("activation", ["silu", "gelu_approx"])
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [11008, 13])
def test_gated_pair_matches_gemvs_and_activation(ctx, orc, kind, m, activation):
    """vtb_hip_segment_matmul_gated_<kind>: act(W_gate x) * (W_up x) in one
    launch against the oracle's GEMVs and math.swiglu / gegluApprox.  Bar:
    the GEMV bar carried through the activation, |d act*u| <= 1.1 |u| dg +
    |act| du with dg, du <= 1e-5 * cond, plus 1e-6 of the output's scale for
    the activation's own rounding."""
    k = 1024 if kind == "q8_0" else 2048
    rng = np.random.default_rng(m + len(kind))
    x = ((rng.random(k, dtype=np.float32) - 0.5) * 2.0).astype(np.float32)
    wg, wu = random_weights(kind, m, k, seed=m), random_weights(kind, m, k, seed=m + 1)
    off_up = (wg.size + 31) // 32 * 32
    blob = np.zeros(off_up + wu.size, np.uint8)
    blob[:wg.size], blob[off_up:] = wg, wu
    wb, xb, ob = ctx.to_device(blob), ctx.to_device(x), ctx.alloc(m * 4)
    with ctx.segment() as seg:
        seg.matmul_gated(kind, ob, wb, 0, off_up, xb, m, k, activation)
    got = ctx.download(ob, np.float32, m).astype(np.float64)
    g = orc.matmul_quant(kind, wg, x, m, k)
    u = orc.matmul_quant(kind, wu, x, m, k)
    ref = (orc.swiglu(g, u) if activation == "silu" else orc.geglu_approx(g, u)).astype(np.float64)
    xa = np.abs(x.astype(np.float64))
    cg = np.abs(np_dequant(kind, wg).astype(np.float64).reshape(m, k)) @ xa
    cu = np.abs(np_dequant(kind, wu).astype(np.float64).reshape(m, k)) @ xa
    bar = 1e-5 * (1.1 * np.abs(u) * cg + (np.abs(g) + 1.0) * cu) + 1e-6 * np.max(np.abs(ref))
    assert np.all(np.abs(got - ref) <= bar), f"{kind} m{m} {activation}"
