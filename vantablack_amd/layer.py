"""Full-GPU decode layer: the host side of vantablack's gpuLayerStep
(src/runtime/forward.zig:419-513) and gpuFinalStep (:515-520), composed from
this library's segment ops.  Per layer and token, on one segment:

  rmsnorm(xb <- x)                          vtb_hip_segment_rmsnorm
  q, k_cur, v_cur = Wq xb, Wk xb, Wv xb     vtb_hip_segment_matmul_<kind>
  RoPE(q, k_cur) + K/V slot write +         vtb_hip_segment_attn_decode_rope_append
    decode attention (one launch)           (the reference's rope x2, copy x2
                                            and three attention kernels)
  xb2 = Wo attn_out; x += xb2               matmul, vtb_hip_segment_residual_add
  rmsnorm(xb <- x); gate, up = Wg xb, Wu xb
  gate = swiglu(gate, up) | gelu_approx     vtb_hip_segment_swiglu / _gelu_approx
  ffn_out = Wd gate; x += ffn_out

gpu_token_step runs a whole token (every layer, then the final step) with
each residual add fused into the rmsnorm that follows it
(vtb_hip_segment_residual_add_rmsnorm), the Q/K/V GEMVs grouped into one
launch (vtb_hip_segment_matmul3_<kind>) and the gate/up GEMVs with the
activation in one launch (vtb_hip_segment_matmul_gated_<kind>) when the
projections share a format: 7 launches per layer instead of 13, the same
arithmetic per output.

The sliding window is the reference's caller-side offset shift
(forward.zig:470-480): the K/V base moves to the window's first row and the
attended length shrinks, and the append lands at row pos either way.  The
weights live in one device buffer at per-tensor byte offsets, as the
reference's weightsBuf()/weightOffset() addresses them (norm weights f32,
projections GGUF-quantised).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

from . import hip

NO_WINDOW = hip.NO_WINDOW
KV_BYTES = {hip.F32: 4, hip.F16: 2, hip.BF16: 2}


@dataclass
class LayerConfig:
    """The LlamaConfig fields a decode layer reads (src/runtime/model.zig:40-70)."""
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    max_seq: int
    rms_eps: float = 1e-5
    rope_base: float = 10000.0
    rope_half: bool = False
    activation: str = "silu"          # or "gelu_approx" (Gemma)
    sliding_window: int = NO_WINDOW
    kv_dtype: int = hip.F16


@dataclass
class LayerOffsets:
    """Byte offsets of one layer's tensors in the weights buffer and the
    quant kind of each projection."""
    attn_norm: int
    wq: int
    wk: int
    wv: int
    wo: int
    ffn_norm: int
    wgate: int
    wup: int
    wdown: int
    kind_q: str
    kind_k: str
    kind_v: str
    kind_o: str
    kind_gate: str
    kind_up: str
    kind_down: str


class LayerScratch:
    """The device activations the layer steps through (MetalBackend's x, xb,
    xb2, q, k_cur, v_cur, attn_out, gate, up, ffn_out, logits)."""

    def __init__(self, ctx, c: LayerConfig, vocab_size: int = 0):
        kv_dim = c.n_kv_heads * c.head_dim
        q_dim = c.n_heads * c.head_dim
        self.x = ctx.alloc(c.dim * 4)
        self.xb = ctx.alloc(max(c.dim, q_dim) * 4)
        self.xb2 = ctx.alloc(c.dim * 4)
        self.q = ctx.alloc(q_dim * 4)
        self.k_cur = ctx.alloc(kv_dim * 4)
        self.v_cur = ctx.alloc(kv_dim * 4)
        self.attn_out = ctx.alloc(q_dim * 4)
        self.gate = ctx.alloc(c.ffn_dim * 4)
        self.up = ctx.alloc(c.ffn_dim * 4)
        self.ffn_out = ctx.alloc(c.dim * 4)
        self.logits = ctx.alloc(vocab_size * 4) if vocab_size else None

    def release(self):
        for b in (self.x, self.xb, self.xb2, self.q, self.k_cur, self.v_cur, self.attn_out, self.gate, self.up,
                  self.ffn_out, self.logits):
            if b is not None:
                b.release()


ACTIVATIONS = ("silu", "gelu_approx")


def _check(c: LayerConfig, pos: int, n_tokens: int = 1):
    """Every config check, before the first launch is encoded: a bad config
    leaves the residual stream and the cache untouched."""
    if c.n_heads * c.head_dim != c.dim:
        raise ValueError("n_heads * head_dim must equal dim (as forward.zig:441-510 assumes)")
    if c.activation not in ACTIVATIONS:
        raise ValueError(f"unknown activation {c.activation!r}")
    if pos + n_tokens > c.max_seq:
        raise ValueError("position beyond max_seq (KvCacheFull)")


def _attention(seg, s, weights, off, kv_k, kv_v, c, layer, pos, grouped=False):
    """Q/K/V GEMVs (one grouped launch when grouped and the three share a
    format), then RoPE + K/V slot write + attention in one launch."""
    kv_dim = c.n_kv_heads * c.head_dim
    row_bytes = kv_dim * KV_BYTES[c.kv_dtype]
    layer_off = layer * c.max_seq * row_bytes
    wstart = 0 if (c.sliding_window == NO_WINDOW or pos < c.sliding_window) else pos - c.sliding_window + 1
    win_off = layer_off + wstart * row_bytes
    if grouped and off.kind_q == off.kind_k == off.kind_v:
        seg.matmul3(off.kind_q, weights, s.xb, c.dim,
                    [(s.q, off.wq, c.dim), (s.k_cur, off.wk, kv_dim), (s.v_cur, off.wv, kv_dim)])
    else:
        seg.matmul_quant(off.kind_q, s.q, weights, off.wq, s.xb, c.dim, c.dim)
        seg.matmul_quant(off.kind_k, s.k_cur, weights, off.wk, s.xb, kv_dim, c.dim)
        seg.matmul_quant(off.kind_v, s.v_cur, weights, off.wv, s.xb, kv_dim, c.dim)
    seg.attn_decode_rope_append(s.attn_out, s.q, kv_k, win_off, kv_v, win_off, s.k_cur, s.v_cur, c.n_heads,
                                c.n_kv_heads, c.head_dim, pos + 1 - wstart, 1.0 / math.sqrt(c.head_dim),
                                c.kv_dtype, pos, c.rope_base, c.rope_half)


def _ffn(seg, s, weights, off, c, grouped=False):
    """gate/up GEMVs and the gated activation (one gated launch when grouped
    and the two share a format), then the down GEMV into s.ffn_out."""
    if grouped and off.kind_gate == off.kind_up:
        # gate/up GEMVs and the activation in one launch, into s.gate
        seg.matmul_gated(off.kind_gate, s.gate, weights, off.wgate, off.wup, s.xb, c.ffn_dim, c.dim, c.activation)
        seg.matmul_quant(off.kind_down, s.ffn_out, weights, off.wdown, s.gate, c.dim, c.ffn_dim)
        return
    seg.matmul_quant(off.kind_gate, s.gate, weights, off.wgate, s.xb, c.ffn_dim, c.dim)
    seg.matmul_quant(off.kind_up, s.up, weights, off.wup, s.xb, c.ffn_dim, c.dim)
    if c.activation == "silu":
        seg.swiglu(s.gate, s.up, c.ffn_dim)
    else:
        seg.gelu_approx(s.gate, s.up, c.ffn_dim)
    seg.matmul_quant(off.kind_down, s.ffn_out, weights, off.wdown, s.gate, c.dim, c.ffn_dim)


def gpu_token_step(seg, s: LayerScratch, weights, offs, kv_k, kv_v, c: LayerConfig, pos: int,
                   output_norm_off: int, output_off: int, output_kind: str, vocab_size: int):
    """Every layer in offs, then gpuFinalStep, for the token at pos (s.x holds
    its embedding); leaves the normalised x in s.x and the logits in s.logits.
    Each residual add runs fused with the rmsnorm after it, and Q/K/V and
    gate/up (+ activation) run grouped when their formats match."""
    _check(c, pos)
    for layer, off in enumerate(offs):
        if layer == 0:
            seg.rmsnorm(s.xb, s.x, weights, off.attn_norm, c.dim, c.rms_eps)
        else:
            seg.residual_add_rmsnorm(s.x, s.ffn_out, s.xb, weights, off.attn_norm, c.dim, c.rms_eps)
        _attention(seg, s, weights, off, kv_k, kv_v, c, layer, pos, grouped=True)
        seg.matmul_quant(off.kind_o, s.xb2, weights, off.wo, s.attn_out, c.dim, c.dim)
        seg.residual_add_rmsnorm(s.x, s.xb2, s.xb, weights, off.ffn_norm, c.dim, c.rms_eps)
        _ffn(seg, s, weights, off, c, grouped=True)
    if offs:
        seg.residual_add_rmsnorm(s.x, s.ffn_out, s.x, weights, output_norm_off, c.dim, c.rms_eps)
    else:
        seg.rmsnorm(s.x, s.x, weights, output_norm_off, c.dim, c.rms_eps)
    seg.matmul_quant(output_kind, s.logits, weights, output_off, s.x, vocab_size, c.dim)


def gpu_layer_step(seg, s: LayerScratch, weights, off: LayerOffsets, kv_k, kv_v, c: LayerConfig, layer: int,
                   pos: int):
    """One decode layer for the token at position pos (cache rows [0, pos)
    already hold the earlier tokens); updates s.x in place and writes row pos
    of this layer's K/V slab.  kv_k / kv_v are layer-major caches of
    c.kv_dtype, [n_layers][max_seq][n_kv_heads][head_dim]."""
    _check(c, pos)
    seg.rmsnorm(s.xb, s.x, weights, off.attn_norm, c.dim, c.rms_eps)
    _attention(seg, s, weights, off, kv_k, kv_v, c, layer, pos)
    seg.matmul_quant(off.kind_o, s.xb2, weights, off.wo, s.attn_out, c.dim, c.dim)
    seg.residual_add(s.x, s.xb2, c.dim)
    seg.rmsnorm(s.xb, s.x, weights, off.ffn_norm, c.dim, c.rms_eps)
    _ffn(seg, s, weights, off, c)
    seg.residual_add(s.x, s.ffn_out, c.dim)


def gpu_final_step(seg, s: LayerScratch, weights, output_norm_off: int, output_off: int, output_kind: str,
                   c: LayerConfig, vocab_size: int):
    """gpuFinalStep (forward.zig:515-520): x = rmsnorm(x) in place, then the
    logits projection into s.logits."""
    seg.rmsnorm(s.x, s.x, weights, output_norm_off, c.dim, c.rms_eps)
    seg.matmul_quant(output_kind, s.logits, weights, output_off, s.x, vocab_size, c.dim)


class PrefillScratch:
    """Device activations of a B-token prefill (prefill.zig Scratch: x, xb,
    xb2, q, k_cur, v_cur, attn_out, gate, up, ffn_out)."""

    def __init__(self, ctx, c: LayerConfig, B: int):
        kv_dim = c.n_kv_heads * c.head_dim
        q_dim = c.n_heads * c.head_dim
        self.B = B
        self.x = ctx.alloc(B * c.dim * 4)
        self.xb = ctx.alloc(B * c.dim * 4)
        self.xb2 = ctx.alloc(B * c.dim * 4)
        self.q = ctx.alloc(B * q_dim * 4)
        self.k_cur = ctx.alloc(B * kv_dim * 4)
        self.v_cur = ctx.alloc(B * kv_dim * 4)
        self.attn_out = ctx.alloc(B * q_dim * 4)
        self.gate = ctx.alloc(B * c.ffn_dim * 4)
        self.up = ctx.alloc(B * c.ffn_dim * 4)
        self.ffn_out = ctx.alloc(B * c.dim * 4)

    def release(self):
        for b in (self.x, self.xb, self.xb2, self.q, self.k_cur, self.v_cur, self.attn_out, self.gate,
                  self.up, self.ffn_out):
            b.release()


def gpu_prefill_layer(seg, s: PrefillScratch, weights, off: LayerOffsets, kv_k, kv_v, c: LayerConfig, layer: int,
                      pos0: int):
    """prefillLayer (src/runtime/prefill.zig:151-231) on the GPU for the B
    tokens at positions pos0 .. pos0+B-1 (s.x holds their embeddings, [B][dim]):
    per-token rmsnorm, batched Q/K/V projections (MFMA; one activation
    pre-pass when they share a format, as gate/up below), RoPE per (token,
    head), the B K/V rows written at pos0, causal attention (MFMA for f16/bf16
    caches), O projection + residual, per-token rmsnorm, batched gate/up, the
    activation, batched down projection + residual.  Updates s.x in place."""
    B = s.B
    _check(c, pos0, B)
    kv_dim = c.n_kv_heads * c.head_dim
    row_bytes = kv_dim * KV_BYTES[c.kv_dtype]
    layer_off = layer * c.max_seq * row_bytes
    seg.rmsnorm_rows(s.xb, s.x, weights, off.attn_norm, c.dim, B, c.rms_eps)
    if off.kind_q == off.kind_k == off.kind_v:
        seg.matmul_batched3(off.kind_q, weights, s.xb, c.dim, B,
                            [(s.q, off.wq, c.dim), (s.k_cur, off.wk, kv_dim), (s.v_cur, off.wv, kv_dim)])
    else:
        seg.matmul_batched(off.kind_q, s.q, weights, off.wq, s.xb, c.dim, c.dim, B)
        seg.matmul_batched(off.kind_k, s.k_cur, weights, off.wk, s.xb, kv_dim, c.dim, B)
        seg.matmul_batched(off.kind_v, s.v_cur, weights, off.wv, s.xb, kv_dim, c.dim, B)
    seg.rope_rows(s.q, B, c.n_heads, c.head_dim, pos0, c.rope_base, c.rope_half)
    seg.rope_rows(s.k_cur, B, c.n_kv_heads, c.head_dim, pos0, c.rope_base, c.rope_half)
    seg.kv_append(kv_k, layer_off + pos0 * row_bytes, c.kv_dtype, s.k_cur, 0, B * kv_dim)
    seg.kv_append(kv_v, layer_off + pos0 * row_bytes, c.kv_dtype, s.v_cur, 0, B * kv_dim)
    seg.attn_prefill(s.attn_out, s.q, kv_k, kv_v, layer_off, B, pos0, c.sliding_window, c.n_heads, c.n_kv_heads,
                     c.head_dim, 1.0 / math.sqrt(c.head_dim), c.kv_dtype)
    seg.matmul_batched(off.kind_o, s.xb2, weights, off.wo, s.attn_out, c.dim, c.dim, B)
    seg.residual_add(s.x, s.xb2, B * c.dim)
    seg.rmsnorm_rows(s.xb, s.x, weights, off.ffn_norm, c.dim, B, c.rms_eps)
    if off.kind_gate == off.kind_up:
        seg.matmul_batched3(off.kind_gate, weights, s.xb, c.dim, B,
                            [(s.gate, off.wgate, c.ffn_dim), (s.up, off.wup, c.ffn_dim)])
    else:
        seg.matmul_batched(off.kind_gate, s.gate, weights, off.wgate, s.xb, c.ffn_dim, c.dim, B)
        seg.matmul_batched(off.kind_up, s.up, weights, off.wup, s.xb, c.ffn_dim, c.dim, B)
    if c.activation == "silu":
        seg.swiglu(s.gate, s.up, B * c.ffn_dim)
    else:
        seg.gelu_approx(s.gate, s.up, B * c.ffn_dim)
    seg.matmul_batched(off.kind_down, s.ffn_out, weights, off.wdown, s.gate, c.dim, c.ffn_dim, B)
    seg.residual_add(s.x, s.ffn_out, B * c.dim)
