"""Host-side mirror of vantablack's attention interface over the HIP C ABI.

Every call goes through ``libvtb_hip.so`` (include/vtb_hip.h).  There is no
CPU fallback: importing this module without the built library, or creating a
Context without a gfx950 device, raises.

Mirrors, by reference file:
  * ``Context`` / ``Buffer`` / ``Segment``  -- src/metal/bridge.zig Device /
    Buf / Segment (externs :16-81, segmentBegin/waitIdle :286-296);
  * ``KvCache``                            -- src/runtime/kv_cache.zig KvCache,
    in device-handle mode (no host slices: memory is discrete HBM);
  * ``LlamaConfig``                        -- the attention fields of
    src/runtime/model.zig LlamaConfig (:40-70);
  * ``layer_attention``                    -- KV write + cpuAttention
  * ``layer_attention_rope``               -- RoPE + KV write + cpuAttention
    (src/runtime/forward.zig:267-270, :187-228);
  * ``prefill_attention``                  -- prefill KV write + the
    ``for b: attentionCausal`` loop (src/runtime/prefill.zig:174-197);
  * ``HipAttentionBackend`` / ``step_attention`` -- the Backend vtable
    (src/runtime/backend.zig:67-133) and stepWithBackend's layer loop
    (forward.zig:152-172), restricted to the attention path.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
import weakref

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# VTB_HIP_LIB selects another build of the same library (tuning variants).
LIB_PATH = os.environ.get("VTB_HIP_LIB") or os.path.join(_HERE, "libvtb_hip.so")

OK, EINVAL, EDEVICE, EFULL, ESHRINK, EUNSUPPORTED = 0, 1, 2, 3, 4, 5
F32, F16, BF16 = 0, 1, 2
DTYPES = {"f32": F32, "f16": F16, "bf16": BF16}
DTYPE_BYTES = {F32: 4, F16: 2, BF16: 2}
NO_WINDOW = (1 << 64) - 1  # maxInt(usize)


class HipError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"[rc={rc}] {msg}")
        self.rc = rc


class KvCacheFull(HipError):
    """forward.zig:27-31 StepError.KvCacheFull."""


class NewMaxSeqBelowPos(HipError):
    """kv_cache.zig:149."""


_ERR_CLASS = {EFULL: KvCacheFull, ESHRINK: NewMaxSeqBelowPos}


class AttnConfigC(ctypes.Structure):
    _fields_ = [("n_heads", ctypes.c_size_t), ("n_kv_heads", ctypes.c_size_t),
                ("head_dim", ctypes.c_size_t), ("max_seq", ctypes.c_size_t),
                ("sliding_window", ctypes.c_size_t)]


# Every symbol include/vtb_hip.h declares, with its ctypes signature.
_P, _S, _I, _F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "vtb_hip_init": ([], _P),
    "vtb_hip_destroy": ([_P], None),
    "vtb_hip_stream": ([_P], _P),
    "vtb_hip_last_error": ([_P], ctypes.c_char_p),
    "vtb_hip_cu_count": ([_P], _I),
    "vtb_hip_xcd_map": ([_P], _I),
    "vtb_hip_xcd_deal": ([_P, _I], _I),
    "vtb_hip_alloc": ([_P, _S], _P),
    "vtb_hip_wrap": ([_P, _P, _S], _P),
    "vtb_hip_release": ([_P], None),
    "vtb_hip_buf_device_ptr": ([_P], _P),
    "vtb_hip_buf_size": ([_P], _S),
    "vtb_hip_upload": ([_P, _P, _S, _P, _S], _I),
    "vtb_hip_download": ([_P, _P, _P, _S, _S], _I),
    "vtb_hip_segment_begin": ([_P], _P),
    "vtb_hip_segment_commit": ([_P], _I),
    "vtb_hip_wait_idle": ([_P], _I),
    "vtb_hip_segment_copy": ([_P, _P, _S, _P, _S, _S], None),
    "vtb_hip_segment_rmsnorm": ([_P, _P, _P, _P, _S, _S, _F], None),
    "vtb_hip_segment_rmsnorm_rows": ([_P, _P, _P, _P, _S, _S, _S, _F], None),
    "vtb_hip_segment_rope_rows": ([_P, _P, _S, _S, _S, _S, _F, _I], None),
    "vtb_hip_segment_swiglu": ([_P, _P, _P, _S], None),
    "vtb_hip_segment_gelu_approx": ([_P, _P, _P, _S], None),
    "vtb_hip_segment_residual_add": ([_P, _P, _P, _S], None),
    "vtb_hip_segment_residual_add_rmsnorm": ([_P, _P, _P, _P, _P, _S, _S, _F], None),
    "vtb_hip_segment_matmul_gated_q8_0": ([_P, _P, _P, _S, _S, _P, _S, _S, _I], None),
    "vtb_hip_segment_matmul_gated_q4_k": ([_P, _P, _P, _S, _S, _P, _S, _S, _I], None),
    "vtb_hip_segment_matmul_gated_q5_k": ([_P, _P, _P, _S, _S, _P, _S, _S, _I], None),
    "vtb_hip_segment_matmul_gated_q6_k": ([_P, _P, _P, _S, _S, _P, _S, _S, _I], None),
    "vtb_hip_segment_matmul_batched3_q8_0": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S, _S], None),
    "vtb_hip_segment_matmul_batched3_q4_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S, _S], None),
    "vtb_hip_segment_matmul_batched3_q5_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S, _S], None),
    "vtb_hip_segment_matmul_batched3_q6_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S, _S], None),
    "vtb_hip_segment_matmul3_q8_0": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S], None),
    "vtb_hip_segment_matmul3_q4_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S], None),
    "vtb_hip_segment_matmul3_q5_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S], None),
    "vtb_hip_segment_matmul3_q6_k": ([_P, _P, _S, _S, _P, _S, _S, _P, _S, _S, _P, _P, _S], None),
    "vtb_hip_segment_kv_append": ([_P, _P, _S, _I, _P, _S, _S], None),
    "vtb_hip_segment_attn_decode": ([_P, _P, _P, _P, _S, _P, _S, _S, _S, _S, _S, _F, _I], None),
    "vtb_hip_segment_attn_decode_append": ([_P, _P, _P, _P, _S, _P, _S, _P, _P, _S, _S, _S, _S, _F, _I], None),
    "vtb_hip_segment_attn_decode_append_noalloc": ([_P, _P, _P, _P, _S, _P, _S, _P, _P, _S, _S, _S, _S, _F, _I],
                                                   None),
    "vtb_hip_segment_attn_decode_rope_append": ([_P, _P, _P, _P, _S, _P, _S, _P, _P, _S, _S, _S, _S, _F, _I,
                                                 _S, _F, _I], None),
    "vtb_hip_segment_attn_prefill": ([_P, _P, _P, _P, _P, _S, _S, _S, _S, _S, _S, _S, _F, _I], None),
    "vtb_hip_kv_cache_init": ([_P, _S, _S, _S, _S, _I], _P),
    "vtb_hip_kv_cache_deinit": ([_P], None),
    "vtb_hip_kv_cache_reset": ([_P], None),
    "vtb_hip_kv_cache_pos": ([_P], _S),
    "vtb_hip_kv_cache_set_pos": ([_P, _S], _I),
    "vtb_hip_kv_cache_max_seq": ([_P], _S),
    "vtb_hip_kv_cache_dtype": ([_P], _I),
    "vtb_hip_kv_cache_advance": ([_P], _I),
    "vtb_hip_kv_cache_slot_offset": ([_P, _S], _S),
    "vtb_hip_kv_cache_layer_offset": ([_P, _S], _S),
    "vtb_hip_kv_cache_k": ([_P], _P),
    "vtb_hip_kv_cache_v": ([_P], _P),
    "vtb_hip_kv_cache_shrink_to_fit": ([_P, _S], _I),
    "vtb_hip_layer_attention": ([_P, _P, ctypes.POINTER(AttnConfigC), _S, _P, _P, _P, _P], _I),
    "vtb_hip_layer_attention_rope": ([_P, _P, ctypes.POINTER(AttnConfigC), _S, _P, _P, _P, _P, _F, _I], _I),
    "vtb_hip_segment_matmul_q8_0": ([_P, _P, _P, _S, _P, _S, _S], None),
    "vtb_hip_matmul_q8_0": ([_P, _P, _P, _S, _P, _S, _S], _I),
    "vtb_hip_segment_matmul_q4_k": ([_P, _P, _P, _S, _P, _S, _S], None),
    "vtb_hip_matmul_q4_k": ([_P, _P, _P, _S, _P, _S, _S], _I),
    "vtb_hip_segment_matmul_q5_k": ([_P, _P, _P, _S, _P, _S, _S], None),
    "vtb_hip_matmul_q5_k": ([_P, _P, _P, _S, _P, _S, _S], _I),
    "vtb_hip_segment_matmul_q6_k": ([_P, _P, _P, _S, _P, _S, _S], None),
    "vtb_hip_matmul_q6_k": ([_P, _P, _P, _S, _P, _S, _S], _I),
    "vtb_hip_segment_matmul_batched_q8_0": ([_P, _P, _P, _S, _P, _S, _S, _S], None),
    "vtb_hip_matmul_batched_q8_0": ([_P, _P, _P, _S, _P, _S, _S, _S], _I),
    "vtb_hip_segment_matmul_batched_q4_k": ([_P, _P, _P, _S, _P, _S, _S, _S], None),
    "vtb_hip_matmul_batched_q4_k": ([_P, _P, _P, _S, _P, _S, _S, _S], _I),
    "vtb_hip_segment_matmul_batched_q5_k": ([_P, _P, _P, _S, _P, _S, _S, _S], None),
    "vtb_hip_matmul_batched_q5_k": ([_P, _P, _P, _S, _P, _S, _S, _S], _I),
    "vtb_hip_segment_matmul_batched_q6_k": ([_P, _P, _P, _S, _P, _S, _S, _S], None),
    "vtb_hip_matmul_batched_q6_k": ([_P, _P, _P, _S, _P, _S, _S, _S], _I),
    "vtb_hip_prefill_attention": ([_P, _P, ctypes.POINTER(AttnConfigC), _S, _S, _P, _P, _P, _P], _I),
    "vtb_hip_reserve": ([_P, ctypes.POINTER(AttnConfigC), _I, _S, _S, _F], _I),
    "vtb_hip_scratch_bytes": ([_P], _S),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libvtb_hip.so.  Raises if it has not been built: the product path
    has no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m vantablack_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = L
    return _lib


def _check(ctx_h, rc: int, what: str):
    if rc != OK:
        msg = lib().vtb_hip_last_error(ctx_h) if ctx_h else b""
        raise _ERR_CLASS.get(rc, HipError)(rc, f"{what}: {(msg or b'').decode()}")


QUANT_KINDS = ("q8_0", "q4_k", "q5_k", "q6_k")


@dataclasses.dataclass
class LlamaConfig:
    """The attention fields of LlamaConfig (model.zig:40-70)."""
    n_heads: int
    n_kv_heads: int
    head_dim: int
    max_seq: int
    sliding_window: int = NO_WINDOW
    rope_base: float = 10000.0  # model.zig:50
    rope_half: bool = False     # model.zig:57

    def c(self) -> AttnConfigC:
        return AttnConfigC(self.n_heads, self.n_kv_heads, self.head_dim, self.max_seq,
                           self.sliding_window)


class Buffer:
    """A VtbHipBuf handle.  Non-owning views (the KvCache's K/V slabs) are
    never released from Python."""

    def __init__(self, ctx: "Context", h: int, keepalive=None, owned: bool = True):
        self.ctx = ctx
        self.h = h
        self._keep = keepalive
        self._owned = owned
        if owned and h:
            ctx._track(self)

    @property
    def ptr(self) -> int:
        return lib().vtb_hip_buf_device_ptr(self.h) or 0

    @property
    def size(self) -> int:
        return int(lib().vtb_hip_buf_size(self.h))

    def release(self):
        if self.h and self._owned:
            lib().vtb_hip_release(self.h)
        self.h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Segment:
    """bridge.zig Segment: encoders enqueue on the context stream; commit()
    reports the first encoding error (it does not wait)."""

    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        self.h = lib().vtb_hip_segment_begin(ctx.h)
        if not self.h:
            raise HipError(EINVAL, "segment_begin failed")

    def copy(self, dst: Buffer, dst_off: int, src: Buffer, src_off: int, n_floats: int):
        lib().vtb_hip_segment_copy(self.h, dst.h, dst_off, src.h, src_off, n_floats)

    def rmsnorm(self, out: Buffer, inp: Buffer, weight: Buffer, weight_off: int, n: int, eps: float):
        """out = rmsnorm(inp) * weight (f32 weights at byte offset weight_off);
        seg.rmsnorm of gpuLayerStep (forward.zig:441)."""
        lib().vtb_hip_segment_rmsnorm(self.h, out.h, inp.h, weight.h, weight_off, n, eps)

    def rmsnorm_rows(self, out: Buffer, inp: Buffer, weight: Buffer, weight_off: int, n: int, rows: int,
                     eps: float):
        lib().vtb_hip_segment_rmsnorm_rows(self.h, out.h, inp.h, weight.h, weight_off, n, rows, eps)

    def rope_rows(self, x: Buffer, rows: int, n_heads: int, head_dim: int, pos0: int, base: float,
                  half: bool = False):
        lib().vtb_hip_segment_rope_rows(self.h, x.h, rows, n_heads, head_dim, pos0, base, 1 if half else 0)

    def swiglu(self, gate: Buffer, up: Buffer, n: int):
        lib().vtb_hip_segment_swiglu(self.h, gate.h, up.h, n)

    def gelu_approx(self, gate: Buffer, up: Buffer, n: int):
        lib().vtb_hip_segment_gelu_approx(self.h, gate.h, up.h, n)

    def residual_add(self, a: Buffer, b: Buffer, n: int):
        lib().vtb_hip_segment_residual_add(self.h, a.h, b.h, n)

    def residual_add_rmsnorm(self, x: Buffer, b: Buffer, out: Buffer, weight: Buffer, weight_off: int, n: int,
                             eps: float):
        """x += b, then out = rmsnorm(x) * weight, in one launch."""
        lib().vtb_hip_segment_residual_add_rmsnorm(self.h, x.h, b.h, out.h, weight.h, weight_off, n, eps)

    def kv_append(self, kv: Buffer, slot_off_bytes: int, kv_dtype: int, src: Buffer, src_off: int, n: int):
        lib().vtb_hip_segment_kv_append(self.h, kv.h, slot_off_bytes, kv_dtype, src.h, src_off, n)

    def attn_decode(self, out: Buffer, q: Buffer, k: Buffer, k_off: int, v: Buffer, v_off: int,
                    n_heads: int, n_kv_heads: int, head_dim: int, seq_len: int, inv_sqrt_hd: float,
                    kv_dtype: int):
        lib().vtb_hip_segment_attn_decode(self.h, out.h, q.h, k.h, k_off, v.h, v_off, n_heads,
                                          n_kv_heads, head_dim, seq_len, inv_sqrt_hd, kv_dtype)

    def attn_decode_append(self, out: Buffer, q: Buffer, k: Buffer, k_off: int, v: Buffer, v_off: int,
                           k_cur: Buffer, v_cur: Buffer, n_heads: int, n_kv_heads: int, head_dim: int,
                           seq_len: int, inv_sqrt_hd: float, kv_dtype: int):
        lib().vtb_hip_segment_attn_decode_append(self.h, out.h, q.h, k.h, k_off, v.h, v_off, k_cur.h, v_cur.h,
                                                 n_heads, n_kv_heads, head_dim, seq_len, inv_sqrt_hd, kv_dtype)

    def attn_decode_append_noalloc(self, out: Buffer, q: Buffer, k: Buffer, k_off: int, v: Buffer, v_off: int,
                                   k_cur: Buffer, v_cur: Buffer, n_heads: int, n_kv_heads: int, head_dim: int,
                                   seq_len: int, inv_sqrt_hd: float, kv_dtype: int):
        """attn_decode_append with the split-K workspace in the decode code
        object's fixed scratch: the call allocates nothing."""
        lib().vtb_hip_segment_attn_decode_append_noalloc(self.h, out.h, q.h, k.h, k_off, v.h, v_off, k_cur.h,
                                                         v_cur.h, n_heads, n_kv_heads, head_dim, seq_len,
                                                         inv_sqrt_hd, kv_dtype)

    def attn_decode_rope_append(self, out: Buffer, q: Buffer, k: Buffer, k_off: int, v: Buffer, v_off: int,
                                k_cur: Buffer, v_cur: Buffer, n_heads: int, n_kv_heads: int, head_dim: int,
                                seq_len: int, inv_sqrt_hd: float, kv_dtype: int, rope_pos: int,
                                rope_base: float, rope_half: bool = False):
        """attn_decode_append with RoPE of q and k_cur at rope_pos fused in
        (the Metal seg.rope x2 + seg.copy x2 + attention, forward.zig:463-483)."""
        lib().vtb_hip_segment_attn_decode_rope_append(self.h, out.h, q.h, k.h, k_off, v.h, v_off, k_cur.h,
                                                      v_cur.h, n_heads, n_kv_heads, head_dim, seq_len,
                                                      inv_sqrt_hd, kv_dtype, rope_pos, rope_base,
                                                      1 if rope_half else 0)

    def matmul_quant(self, kind: str, out: Buffer, w: Buffer, w_offset: int, acts: Buffer, m: int, k: int):
        """out = W @ acts for m rows of `kind` blocks (q8_0, q4_k, q5_k, q6_k):
        segMatmulQuant (forward.zig:400-417) on the segment."""
        if kind not in QUANT_KINDS:
            raise ValueError(f"unknown quant kind {kind!r}")
        getattr(lib(), f"vtb_hip_segment_matmul_{kind}")(self.h, out.h, w.h, w_offset, acts.h, m, k)

    def matmul_gated(self, kind: str, out: Buffer, w: Buffer, w_off_gate: int, w_off_up: int, acts: Buffer, m: int,
                     k: int, activation: str = "silu"):
        """out = act(W_gate @ acts) * (W_up @ acts): the FFN's gate/up GEMVs and
        swiglu (activation "silu") or gegluApprox ("gelu_approx") in one launch."""
        if kind not in QUANT_KINDS:
            raise ValueError(f"unknown quant kind {kind!r}")
        act = {"silu": 0, "gelu_approx": 1}[activation]
        getattr(lib(), f"vtb_hip_segment_matmul_gated_{kind}")(self.h, out.h, w.h, w_off_gate, w_off_up, acts.h, m, k,
                                                               act)

    def matmul_batched3(self, kind: str, w: Buffer, acts: Buffer, k: int, n_tokens: int, blocks):
        """Two or three batched matmuls of one format over the same tokens,
        one activation pre-pass: blocks = [(out, w_offset, m), ...]."""
        if kind not in QUANT_KINDS:
            raise ValueError(f"unknown quant kind {kind!r}")
        if len(blocks) not in (2, 3):
            raise ValueError("matmul_batched3 takes two or three weight blocks")
        b = list(blocks) + ([(None, 0, 0)] if len(blocks) == 2 else [])
        args = []
        for out, off, m in b:
            args += [out.h if out is not None else None, off, m]
        getattr(lib(), f"vtb_hip_segment_matmul_batched3_{kind}")(self.h, *args, w.h, acts.h, k, n_tokens)

    def matmul3(self, kind: str, w: Buffer, acts: Buffer, k: int, blocks):
        """Two or three GEMVs of one format over the same acts in one launch:
        blocks = [(out, w_offset, m), ...]."""
        if kind not in QUANT_KINDS:
            raise ValueError(f"unknown quant kind {kind!r}")
        if len(blocks) not in (2, 3):
            raise ValueError("matmul3 takes two or three row blocks")
        b = list(blocks) + ([(None, 0, 0)] if len(blocks) == 2 else [])
        args = []
        for out, off, m in b:
            args += [out.h if out is not None else None, off, m]
        getattr(lib(), f"vtb_hip_segment_matmul3_{kind}")(self.h, *args, w.h, acts.h, k)

    def matmul_batched(self, kind: str, out: Buffer, w: Buffer, w_offset: int, acts: Buffer, m: int, k: int,
                       n_tokens: int):
        """out[b] = W @ acts[b] for n_tokens tokens (prefill.zig matmulBatched)
        on the segment; acts f32 [n_tokens][k], out f32 [n_tokens][m]."""
        if kind not in QUANT_KINDS:
            raise ValueError(f"unknown quant kind {kind!r}")
        getattr(lib(), f"vtb_hip_segment_matmul_batched_{kind}")(self.h, out.h, w.h, w_offset, acts.h, m, k,
                                                                  n_tokens)

    def attn_prefill(self, out: Buffer, q: Buffer, k: Buffer, v: Buffer, layer_off: int, n_tokens: int,
                     pos0: int, sliding_window: int, n_heads: int, n_kv_heads: int, head_dim: int,
                     inv_sqrt_hd: float, dtype: int):
        lib().vtb_hip_segment_attn_prefill(self.h, out.h, q.h, k.h, v.h, layer_off, n_tokens, pos0,
                                           sliding_window, n_heads, n_kv_heads, head_dim, inv_sqrt_hd,
                                           dtype)

    def commit(self):
        h, self.h = self.h, None
        if h:
            _check(self.ctx.h, lib().vtb_hip_segment_commit(h), "segment_commit")

    def __enter__(self):
        return self

    def __exit__(self, et, ev, tb):
        if self.h:
            if et is None:
                self.commit()
            else:
                lib().vtb_hip_segment_commit(self.h)
                self.h = None


class Context:
    """bridge.zig Device: process-long; owns one HIP stream."""

    def __init__(self):
        self.h = lib().vtb_hip_init()
        if not self.h:
            raise HipError(EDEVICE, "vtb_hip_init failed: no gfx950 device or code objects did not load")
        self._owned = weakref.WeakSet()

    def _track(self, obj):
        self._owned.add(obj)

    @property
    def stream(self) -> int:
        return lib().vtb_hip_stream(self.h) or 0

    @property
    def cu_count(self) -> int:
        return int(lib().vtb_hip_cu_count(self.h))

    @property
    def xcd_map(self) -> int:
        """XCDs the decode launches' workgroups are dealt over (0: no
        XCD-local split merge)."""
        return int(lib().vtb_hip_xcd_map(self.h))

    @property
    def last_error(self) -> str:
        return (lib().vtb_hip_last_error(self.h) or b"").decode()

    def alloc(self, nbytes: int) -> Buffer:
        h = lib().vtb_hip_alloc(self.h, nbytes)
        if not h:
            raise HipError(EDEVICE, f"alloc({nbytes}) failed: {self.last_error}")
        return Buffer(self, h)

    def wrap(self, device_ptr: int, nbytes: int, keepalive=None) -> Buffer:
        h = lib().vtb_hip_wrap(self.h, device_ptr, nbytes)
        if not h:
            raise HipError(EINVAL, "wrap failed")
        return Buffer(self, h, keepalive)

    def wrap_tensor(self, t) -> Buffer:
        """Wrap a contiguous torch device tensor (no copy; the tensor is kept
        alive by the Buffer)."""
        assert t.is_cuda and t.is_contiguous()
        return self.wrap(t.data_ptr(), t.numel() * t.element_size(), keepalive=t)

    def upload(self, buf: Buffer, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        _check(self.h, lib().vtb_hip_upload(self.h, buf.h, offset, a.ctypes.data, a.nbytes), "upload")

    def download(self, buf: Buffer, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(self.h, lib().vtb_hip_download(self.h, out.ctypes.data, buf.h, offset, out.nbytes), "download")
        return out

    def to_device(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes, 16))
        self.upload(b, a)
        return b

    def segment(self) -> Segment:
        return Segment(self)

    def wait_idle(self):
        _check(self.h, lib().vtb_hip_wait_idle(self.h), "wait_idle")

    def reserve(self, cfg, kv_dtype, max_batch: int, max_matmul_k: int = 0, rope_base: float = 0.0):
        """vtb_hip_reserve: grow every on-demand scratch buffer once (prefill.zig
        Scratch.init's sizing), so later calls within the bounds allocate
        nothing.  cfg is an AttnConfigC or anything with its five fields."""
        c = cfg if isinstance(cfg, AttnConfigC) else AttnConfigC(
            cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq, cfg.sliding_window)
        dt = DTYPES[kv_dtype] if isinstance(kv_dtype, str) else kv_dtype
        _check(self.h, lib().vtb_hip_reserve(self.h, ctypes.byref(c), dt, max_batch, max_matmul_k, rope_base),
               "reserve")

    @property
    def scratch_bytes(self) -> int:
        return int(lib().vtb_hip_scratch_bytes(self.h))

    def close(self):
        """Release every buffer and cache still alive on this context, then
        destroy it (vtb_hip_destroy)."""
        if self.h:
            for obj in list(self._owned):
                obj.close() if isinstance(obj, KvCache) else obj.release()
            lib().vtb_hip_destroy(self.h)
            self.h = None


class KvCache:
    """kv_cache.zig KvCache in device-handle mode: layer-major
    [n_layers][max_seq][n_kv_heads][head_dim] of `dtype` in HBM."""

    def __init__(self, ctx: Context, n_layers: int, n_kv_heads: int, head_dim: int, max_seq: int,
                 dtype="f32"):
        self.ctx = ctx
        self.dtype = DTYPES[dtype] if isinstance(dtype, str) else dtype
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.h = lib().vtb_hip_kv_cache_init(ctx.h, n_layers, n_kv_heads, head_dim, max_seq, self.dtype)
        if not self.h:
            raise HipError(EDEVICE, f"kv_cache_init failed: {ctx.last_error}")
        ctx._track(self)

    @property
    def pos(self) -> int:
        return int(lib().vtb_hip_kv_cache_pos(self.h))

    @pos.setter
    def pos(self, p: int):
        _check(self.ctx.h, lib().vtb_hip_kv_cache_set_pos(self.h, p), "set_pos")

    @property
    def max_seq(self) -> int:
        return int(lib().vtb_hip_kv_cache_max_seq(self.h))

    @property
    def row_elems(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def elem_bytes(self) -> int:
        return DTYPE_BYTES[self.dtype]

    def reset(self):
        lib().vtb_hip_kv_cache_reset(self.h)

    def advance(self):
        rc = lib().vtb_hip_kv_cache_advance(self.h)
        if rc == EFULL:
            raise KvCacheFull(rc, "advance past max_seq")
        _check(self.ctx.h, rc, "advance")

    def slot_offset(self, layer: int) -> int:
        off = lib().vtb_hip_kv_cache_slot_offset(self.h, layer)
        if off == NO_WINDOW:
            raise IndexError("slot out of range")
        return int(off)

    def layer_offset(self, layer: int) -> int:
        off = lib().vtb_hip_kv_cache_layer_offset(self.h, layer)
        if off == NO_WINDOW:
            raise IndexError("layer out of range")
        return int(off)

    @property
    def k(self) -> Buffer:
        return Buffer(self.ctx, lib().vtb_hip_kv_cache_k(self.h), owned=False)

    @property
    def v(self) -> Buffer:
        return Buffer(self.ctx, lib().vtb_hip_kv_cache_v(self.h), owned=False)

    def shrink_to_fit(self, new_max_seq: int):
        _check(self.ctx.h, lib().vtb_hip_kv_cache_shrink_to_fit(self.h, new_max_seq), "shrink_to_fit")

    # --- host access (explicit copies; the reference's host slices do not exist here)
    def _np_dtype(self):
        return np.float32 if self.dtype == F32 else np.uint16

    def read_rows(self, which: str, layer: int, n_rows: int) -> np.ndarray:
        """keysFor/valuesFor (kv_cache.zig:116-128) as a host copy:
        [n_rows, n_kv_heads, head_dim] in storage form (f32 or u16 bits)."""
        buf = self.k if which == "k" else self.v
        out = self.ctx.download(buf, self._np_dtype(), n_rows * self.row_elems, self.layer_offset(layer))
        return out.reshape(n_rows, self.n_kv_heads, self.head_dim)

    def write_rows(self, which: str, layer: int, row0: int, data: np.ndarray):
        """Upload storage-form rows [n, n_kv_heads, head_dim] starting at row0."""
        buf = self.k if which == "k" else self.v
        d = np.ascontiguousarray(data, dtype=self._np_dtype())
        self.ctx.upload(buf, d, self.layer_offset(layer) + row0 * self.row_elems * self.elem_bytes)

    def close(self):
        if self.h:
            lib().vtb_hip_kv_cache_deinit(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def layer_attention(seg: Segment, cache: KvCache, c: LlamaConfig, layer: int, q: Buffer,
                    k_cur: Buffer, v_cur: Buffer, attn_out: Buffer):
    """forward.zig:267-270 + cpuAttention (:187-228) for one layer: write
    k_cur/v_cur into the slot at cache.pos, then attend [window_start, pos]."""
    cc = c.c()
    _check(seg.ctx.h, lib().vtb_hip_layer_attention(seg.h, cache.h, ctypes.byref(cc), layer, q.h, k_cur.h,
                                                    v_cur.h, attn_out.h), "layer_attention")


def layer_attention_rope(seg: Segment, cache: KvCache, c: LlamaConfig, layer: int, q: Buffer,
                         k_cur: Buffer, v_cur: Buffer, attn_out: Buffer):
    """forward.zig:250-270 + cpuAttention for one layer: RoPE of q and k_cur
    at cache.pos (math.rope, or math.ropeHalf when c.rope_half), the slot
    write and the attention, in one launch.  q and k_cur are left unrotated."""
    cc = c.c()
    _check(seg.ctx.h, lib().vtb_hip_layer_attention_rope(seg.h, cache.h, ctypes.byref(cc), layer, q.h, k_cur.h,
                                                         v_cur.h, attn_out.h, c.rope_base,
                                                         1 if c.rope_half else 0), "layer_attention_rope")


def prefill_attention(seg: Segment, cache: KvCache, c: LlamaConfig, layer: int, n_tokens: int, q: Buffer,
                      k_cur: Buffer, v_cur: Buffer, attn_out: Buffer):
    """prefill.zig:174-197 for one layer: write n_tokens K/V rows at
    cache.pos.., then causal attention for every query."""
    cc = c.c()
    _check(seg.ctx.h, lib().vtb_hip_prefill_attention(seg.h, cache.h, ctypes.byref(cc), layer, n_tokens, q.h,
                                                      k_cur.h, v_cur.h, attn_out.h), "prefill_attention")


@dataclasses.dataclass
class Capabilities:
    """backend.zig:43-55."""
    supports_fused_qkv: bool = False
    supports_kquant_gpu: bool = False
    supports_mlx_q4: bool = False
    unified_memory: bool = False
    name: str = "hip"


class HipAttentionBackend:
    """The attention half of a hybrid backend (backend_cpu.zig:34-49 pattern):
    layer_step writes the KV slot and runs decode attention on the GPU;
    finalize_token is the only host-visibility point (backend.zig:86-88)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self._seg = None

    def layer_step(self, cache: KvCache, c: LlamaConfig, layer: int, q: Buffer, k_cur: Buffer,
                   v_cur: Buffer, attn_out: Buffer, rope: bool = False):
        """rope=False: q / k_cur are already rotated (forward.zig:250-265 ran
        on the host); rope=True: they are not, and RoPE is fused in."""
        if self._seg is None:
            self._seg = self.ctx.segment()
        if rope:
            layer_attention_rope(self._seg, cache, c, layer, q, k_cur, v_cur, attn_out)
        else:
            layer_attention(self._seg, cache, c, layer, q, k_cur, v_cur, attn_out)

    def finalize_token(self):
        if self._seg is not None:
            seg, self._seg = self._seg, None
            seg.commit()
        self.ctx.wait_idle()

    def capabilities(self) -> Capabilities:
        return Capabilities()


def step_attention(be: HipAttentionBackend, cache: KvCache, c: LlamaConfig, layer_io):
    """stepWithBackend's layer loop (forward.zig:152-172) restricted to the
    attention path: KvCacheFull guard, one layer_step per layer, one advance,
    then finalize_token.  layer_io[l] = (q, k_cur, v_cur, attn_out)."""
    if cache.pos >= c.max_seq:
        raise KvCacheFull(EFULL, "KvCacheFull")
    for layer, (q, k_cur, v_cur, out) in enumerate(layer_io):
        be.layer_step(cache, c, layer, q, k_cur, v_cur, out)
    cache.advance()
    be.finalize_token()
