"""Host logic of vantablack_amd.layer without a GPU: a recording stand-in for
the segment checks that gpu_layer_step encodes gpuLayerStep's sequence
(src/runtime/forward.zig:441-510, with the reference's rope x2 + copy x2 +
attention trio as the one fused attention launch), gpu_final_step
gpuFinalStep's (:517-518), gpu_token_step its 7 launches per layer, and
gpu_prefill_layer prefillLayer's order (src/runtime/prefill.zig:151-231);
and that the guards raise."""
import pytest

from vantablack_amd import hip
from vantablack_amd.layer import (LayerConfig, LayerOffsets, gpu_final_step, gpu_layer_step, gpu_prefill_layer,
                                  gpu_token_step)


class Recorder:
    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def rec(*args):
            self.calls.append((name, args))
        return rec


class Buf:
    def __init__(self, name):
        self.name = name


class Scratch:
    def __init__(self, B=1):
        for n in ("x", "xb", "xb2", "q", "k_cur", "v_cur", "attn_out", "gate", "up", "ffn_out", "logits"):
            setattr(self, n, Buf(n))
        self.B = B


def _off(kind="q4_k", down="q4_k"):
    return LayerOffsets(0, 100, 200, 300, 400, 500, 600, 700, 800, kind, kind, kind, kind, kind, kind, down)


C = LayerConfig(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, max_seq=32, kv_dtype=hip.F16)


def test_layer_step_is_the_reference_encoder_sequence():
    seg = Recorder()
    gpu_layer_step(seg, Scratch(), Buf("w"), _off(), Buf("k"), Buf("v"), C, 1, 5)
    names = [n for n, _ in seg.calls]
    assert names == ["rmsnorm", "matmul_quant", "matmul_quant", "matmul_quant", "attn_decode_rope_append",
                     "matmul_quant", "residual_add", "rmsnorm", "matmul_quant", "matmul_quant", "swiglu",
                     "matmul_quant", "residual_add"]
    att = dict(seg.calls)["attn_decode_rope_append"]
    row_bytes = C.n_kv_heads * C.head_dim * 2
    assert att[3] == 1 * C.max_seq * row_bytes  # layer 1's K slab, no window
    assert att[11] == 6 and att[14] == 5       # attended rows pos + 1, RoPE at pos


def test_window_shifts_the_base_and_shortens_the_range():
    seg = Recorder()
    c = LayerConfig(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, max_seq=32, sliding_window=4,
                    kv_dtype=hip.F16)
    gpu_layer_step(seg, Scratch(), Buf("w"), _off(), Buf("k"), Buf("v"), c, 0, 10)
    att = dict(seg.calls)["attn_decode_rope_append"]
    assert att[3] == (10 - 4 + 1) * 2 * 64 * 2 and att[11] == 4  # forward.zig:470-480


def test_final_step_and_token_step_launches():
    seg = Recorder()
    gpu_final_step(seg, Scratch(), Buf("w"), 900, 1000, "q8_0", C, 77)
    assert [n for n, _ in seg.calls] == ["rmsnorm", "matmul_quant"]
    seg = Recorder()
    gpu_token_step(seg, Scratch(), Buf("w"), [_off(), _off()], Buf("k"), Buf("v"), C, 3, 900, 1000, "q8_0", 77)
    names = [n for n, _ in seg.calls]
    per_layer = ["matmul3", "attn_decode_rope_append", "matmul_quant", "residual_add_rmsnorm", "matmul_gated",
                 "matmul_quant"]
    assert names == ["rmsnorm"] + per_layer + ["residual_add_rmsnorm"] + per_layer + \
        ["residual_add_rmsnorm", "matmul_quant"]
    # mixed formats fall back to single GEMVs and the separate activation
    seg = Recorder()
    gpu_token_step(seg, Scratch(), Buf("w"), [_off("q4_k", "q6_k")], Buf("k"), Buf("v"), C, 0, 900, 1000, "q8_0", 7)
    assert [n for n, _ in seg.calls].count("matmul_gated") == 1
    off = _off()
    off.kind_v = "q6_k"
    seg = Recorder()
    gpu_token_step(seg, Scratch(), Buf("w"), [off], Buf("k"), Buf("v"), C, 0, 900, 1000, "q8_0", 7)
    assert "matmul3" not in [n for n, _ in seg.calls]


def test_prefill_layer_order():
    seg = Recorder()
    gpu_prefill_layer(seg, Scratch(B=8), Buf("w"), _off(), Buf("k"), Buf("v"), C, 0, 4)
    names = [n for n, _ in seg.calls]
    assert names == ["rmsnorm_rows", "matmul_batched3", "rope_rows", "rope_rows", "kv_append", "kv_append",
                     "attn_prefill", "matmul_batched", "residual_add", "rmsnorm_rows",
                     "matmul_batched3", "swiglu", "matmul_batched", "residual_add"]
    # the queries reach the attention as the f32 s.q (prefill.zig:167-197)
    assert dict(seg.calls)["attn_prefill"][1].name == "q"


def test_guards():
    """Every guard raises before the first launch is encoded: a bad config
    leaves the segment, the residual stream and the cache untouched."""
    bad = LayerConfig(dim=200, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, max_seq=32)
    relu = LayerConfig(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, max_seq=32, activation="relu")
    cases = [
        lambda seg: gpu_layer_step(seg, Scratch(), Buf("w"), _off(), Buf("k"), Buf("v"), bad, 0, 0),
        lambda seg: gpu_token_step(seg, Scratch(), Buf("w"), [_off()], Buf("k"), Buf("v"), C, 32, 0, 0, "q8_0", 7),
        lambda seg: gpu_prefill_layer(seg, Scratch(B=30), Buf("w"), _off(), Buf("k"), Buf("v"), C, 0, 4),
        lambda seg: gpu_layer_step(seg, Scratch(), Buf("w"), _off(), Buf("k"), Buf("v"), relu, 0, 0),
        lambda seg: gpu_token_step(seg, Scratch(), Buf("w"), [_off()], Buf("k"), Buf("v"), relu, 0, 0, 0, "q8_0", 7),
        lambda seg: gpu_prefill_layer(seg, Scratch(B=8), Buf("w"), _off(), Buf("k"), Buf("v"), relu, 0, 0),
    ]
    for case in cases:
        seg = Recorder()
        with pytest.raises(ValueError):
            case(seg)
        assert seg.calls == [], [n for n, _ in seg.calls]
