"""Batched quantised matmul (prefill projections) on the GPU, through the C
ABI, against the oracle's restatement of prefill.zig matmulBatched
(dequantToF32 + simd.dot_f32).

Bars: |got - ref| <= 1e-5 * sum_j |W_ij x_bj| per output (holds however much
a sum cancels), and <= 1e-4 relative wherever the sum is not a cancellation
(|ref| > 1e-3 * sum |W||x|) -- the reference's own Metal quant bar
(bridge.zig:466-470).
"""
import numpy as np
import pytest

from tests.quant import np_dequant, random_weights

pytestmark = pytest.mark.gpu
KINDS = ["q8_0", "q4_k", "q5_k", "q6_k"]


def batched_case(ctx, orc, kind, m, k, B, seed, w_offset=0, x=None, rel=True):
    w = random_weights(kind, m, k, seed)
    if x is None:
        x = orc.normal(seed + 1, B * k).reshape(B, k)
    wbuf = ctx.to_device(np.concatenate([np.zeros(w_offset, np.uint8), w]))
    xb, ob = ctx.to_device(np.ascontiguousarray(x, np.float32)), ctx.alloc(B * m * 4)
    with ctx.segment() as seg:
        seg.matmul_batched(kind, ob, wbuf, w_offset, xb, m, k, B)
    got = ctx.download(ob, np.float32, B * m).reshape(B, m).astype(np.float64)
    ref = orc.matmul_batched(kind, w, x, m, k, B).astype(np.float64)
    W = np_dequant(kind, w).astype(np.float64).reshape(m, k)
    cond = np.abs(x.astype(np.float64)) @ np.abs(W).T
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 * cond), f"{kind} m{m} k{k} B{B}: max err/cond {np.max(err / cond):.2e}"
    if rel:
        big = np.abs(ref) > 1e-3 * cond
        assert np.all(err[big] <= 1e-4 * np.abs(ref[big])), f"{kind} m{m} k{k} B{B}: relative error above 1e-4"
    return got


@pytest.mark.parametrize("kind", KINDS)
def test_single_tile(ctx, orc, kind):
    batched_case(ctx, orc, kind, 128, 512, 128, seed=1)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m,k,B", [(1, 256, 1), (37, 512, 5), (300, 1024, 129), (130, 2304, 257)])
def test_ragged_shapes(ctx, orc, kind, m, k, B):
    # rows and tokens not multiples of the 128 tile; k of 1, 2, 4 and 9 blocks
    batched_case(ctx, orc, kind, m, k, B, seed=m + k + B)


@pytest.mark.parametrize("kind", KINDS)
def test_llama3_8b_shape(ctx, orc, kind):
    # C4 projection widths (dim 4096, kv_dim 1024) on a 256-token slice
    batched_case(ctx, orc, kind, 1024, 4096, 256, seed=7)


@pytest.mark.parametrize("kind", KINDS)
def test_weight_offset(ctx, orc, kind):
    batched_case(ctx, orc, kind, 64, 1024, 40, seed=9, w_offset=4100)


def test_activation_extremes(ctx, orc):
    # magnitudes spread over 80 binades and exact zeros: the per-token
    # power-of-two scaling and the two-piece split must hold every value to
    # 22 bits (or 2^-40 of the token's largest).  With this range a sum near
    # 1e-3 of sum |W||x| has lost its small terms in either f32 accumulation
    # order (the oracle's and the GPU's alike), so only the
    # conditioning-relative bar applies.
    rng = np.random.default_rng(3)
    B, k = 64, 1024
    x = (rng.standard_normal((B, k)) * np.exp2(rng.integers(-40, 40, (B, k)))).astype(np.float32)
    x[:, ::7] = 0.0
    for kind in KINDS:
        batched_case(ctx, orc, kind, 96, k, B, seed=11, x=x, rel=False)


def test_rows_agree_with_single_token_gemv(ctx, orc):
    # one token through the batched kernel vs the GEMV kernel: same weights,
    # both within the bar of their own oracle restatements, so within 2e-5 of
    # each other relative to sum |W||x|
    kind, m, k = "q6_k", 256, 2048
    w = random_weights(kind, m, k, 5)
    x = orc.normal(6, k)
    wb, xb = ctx.to_device(w), ctx.to_device(x)
    o1, o2 = ctx.alloc(m * 4), ctx.alloc(m * 4)
    with ctx.segment() as seg:
        seg.matmul_batched(kind, o1, wb, 0, xb, m, k, 1)
        seg.matmul_quant(kind, o2, wb, 0, xb, m, k)
    a = ctx.download(o1, np.float32, m).astype(np.float64)
    b = ctx.download(o2, np.float32, m).astype(np.float64)
    cond = np.abs(np_dequant(kind, w).astype(np.float64).reshape(m, k)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(a - b) <= 2e-5 * cond)


def test_rejections(ctx):
    import vantablack_amd as vb
    w = ctx.alloc(1 << 20)
    x = ctx.alloc(1 << 20)
    o = ctx.alloc(1 << 20)
    for kind, m, k, B, off in [("q4_k", 4, 300, 2, 0),        # k not whole blocks
                               ("q8_0", 4, 64, 2, 2),         # weights not 4-byte aligned
                               ("q8_0", 1, 32800, 1, 0),      # k above MAX_K
                               ("q6_k", 8000, 512, 2, 0)]:    # weights beyond the buffer
        with pytest.raises(vb.HipError):
            with ctx.segment() as seg:
                seg.matmul_batched(kind, o, w, off, x, m, k, B)


def test_synchronous_entry(ctx, orc):
    import vantablack_amd as vb
    kind, m, k, B = "q5_k", 64, 512, 33
    w = random_weights(kind, m, k, seed=12)
    x = orc.normal(13, B * k).reshape(B, k)
    wb, xb, ob = ctx.to_device(w), ctx.to_device(x), ctx.alloc(B * m * 4)
    assert vb.hip.lib().vtb_hip_matmul_batched_q5_k(ctx.h, ob.h, wb.h, 0, xb.h, m, k, B) == 0
    got = ctx.download(ob, np.float32, B * m).reshape(B, m)
    ref = orc.matmul_batched(kind, w, x, m, k, B)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


@pytest.mark.parametrize("kind", ["q8_0", "q4_k", "q5_k", "q6_k"])
def test_shared_prepass_blocks_match_single_calls(ctx, kind):
    """vtb_hip_segment_matmul_batched3_<kind>: three weight blocks over one
    activation pre-pass give exactly what three single batched calls give
    (same kernels, same split of the activations)."""
    k, B, ms = 512, 37, (256, 64, 130)
    rng = np.random.default_rng(len(kind))
    acts = rng.standard_normal((B, k)).astype(np.float32)
    ws = [random_weights(kind, m, k, seed=m) for m in ms]
    offs, pos = [], 0
    for w in ws:
        offs.append(pos)
        pos += (w.size + 31) // 32 * 32
    blob = np.zeros(pos, np.uint8)
    for w, o in zip(ws, offs):
        blob[o:o + w.size] = w
    wb, xb = ctx.to_device(blob), ctx.to_device(acts)
    grouped = [ctx.alloc(B * m * 4) for m in ms]
    single = [ctx.alloc(B * m * 4) for m in ms]
    with ctx.segment() as seg:
        seg.matmul_batched3(kind, wb, xb, k, B, [(o, off, m) for o, off, m in zip(grouped, offs, ms)])
        for o, off, m in zip(single, offs, ms):
            seg.matmul_batched(kind, o, wb, off, xb, m, k, B)
    for g, s1, m in zip(grouped, single, ms):
        assert np.array_equal(ctx.download(g, np.float32, B * m), ctx.download(s1, np.float32, B * m))
