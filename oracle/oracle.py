"""Python face of the CPU parity oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only to check (or time, as the CPU baseline) the
HIP path -- never as the product path.

Contents:
  * ctypes bindings to ``liboracle.so`` (the C restatement in
    ``attn_oracle.c`` of vantablack's ``forward.cpuAttention``
    (src/runtime/forward.zig:187-228), ``prefill.attentionCausal``
    (src/runtime/prefill.zig:237-287), ``math.softmax`` (src/kernels/math.zig:
    136-150), the KvCache layout (src/runtime/kv_cache.zig) and the pool
    (src/runtime/pool.zig));
  * ``math.rope`` / ``math.ropeHalf`` (src/kernels/math.zig:85-133);
  * the quantised matmuls of src/kernels/simd.zig (Q8_0, Q4_K, Q5_K, Q6_K) in
    ``quant_oracle.c``;
  * the portable seeded input generator (SplitMix64 -> f64 Box-Muller -> f32
    -> KV dtype) used for every parity input;
  * exact dtype helpers (f32 -> f16/bf16 round-to-nearest-even, and the exact
    upcasts of src/kernels/simd.zig:123-126 and forward.zig:661-666).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
NO_WINDOW = (1 << 64) - 1  # maxInt(usize): sliding window disabled (model.zig:59-62)


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


class KvCacheC(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_size_t), ("n_kv_heads", ctypes.c_size_t),
                ("head_dim", ctypes.c_size_t), ("max_seq", ctypes.c_size_t),
                ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("pos", ctypes.c_size_t)]


class ConfigC(ctypes.Structure):
    _fields_ = [("n_heads", ctypes.c_size_t), ("n_kv_heads", ctypes.c_size_t),
                ("head_dim", ctypes.c_size_t), ("max_seq", ctypes.c_size_t),
                ("sliding_window", ctypes.c_size_t)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, S, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
        L.vtb_oracle_softmax.argtypes = [P, S]
        L.vtb_oracle_rmsnorm.argtypes = [P, P, S, F]
        L.vtb_oracle_swiglu.argtypes = [P, P, S]
        L.vtb_oracle_geglu_approx.argtypes = [P, P, S]
        L.vtb_oracle_rope.argtypes = [P, S, S, F]
        L.vtb_oracle_quant_block_bytes.argtypes = [ctypes.c_int]
        L.vtb_oracle_quant_block_bytes.restype = S
        L.vtb_oracle_quant_block_elems.argtypes = [ctypes.c_int]
        L.vtb_oracle_quant_block_elems.restype = S
        L.vtb_oracle_dequant_block.argtypes = [ctypes.c_int, P, P]
        L.vtb_oracle_matmul_quant.argtypes = [ctypes.c_int, P, P, P, S, S]
        L.vtb_oracle_matmul_batched.argtypes = [ctypes.c_int, P, P, P, S, S, S]
        L.vtb_oracle_rope_half.argtypes = [P, S, S, F]
        L.vtb_oracle_rope_inv_freq.argtypes = [P, S, F]
        L.vtb_oracle_argmax.argtypes = [P, S]
        L.vtb_oracle_argmax.restype = S
        L.vtb_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.vtb_oracle_f16_to_f32.restype = F
        L.vtb_oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.vtb_oracle_bf16_to_f32.restype = F
        L.vtb_oracle_upcast_f16.argtypes = [P, P, S]
        L.vtb_oracle_upcast_bf16.argtypes = [P, P, S]
        L.vtb_oracle_kv_slot_offset.argtypes = [P, S]
        L.vtb_oracle_kv_slot_offset.restype = S
        L.vtb_oracle_kv_layer_offset.argtypes = [P, S]
        L.vtb_oracle_kv_layer_offset.restype = S
        L.vtb_oracle_kv_advance.argtypes = [P]
        L.vtb_oracle_kv_shrink_to_fit.argtypes = [P, S]
        L.vtb_oracle_window_start.argtypes = [S, S]
        L.vtb_oracle_window_start.restype = S
        L.vtb_oracle_cpu_attention.argtypes = [P, P, P, S, P, P]
        L.vtb_oracle_attention_causal.argtypes = [P, P, P, S, S, P, P]
        L.vtb_oracle_attention_f64.argtypes = [P, P, P, S, S, P]
        L.vtb_oracle_pool_init.argtypes = [S, S]
        L.vtb_oracle_pool_init.restype = P
        L.vtb_oracle_pool_deinit.argtypes = [P]
        L.vtb_oracle_pool_workers.argtypes = [P]
        L.vtb_oracle_pool_workers.restype = S
        L.vtb_oracle_pool_set_active.argtypes = [P, S]
        L.vtb_oracle_pool_sum.argtypes = [P, P, S]
        L.vtb_oracle_pool_sum.restype = ctypes.c_uint64
        L.vtb_oracle_cpu_attention_pooled.argtypes = [P, P, P, P, S, S, P, P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------
# Portable seeded RNG: SplitMix64 (counter-based) -> f64 Box-Muller -> f32.
# ---------------------------------------------------------------------------
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    """Value number ``idx`` of the SplitMix64 stream started at ``seed``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (idx.astype(np.uint64) + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n standard normals (f64 Box-Muller, one normal per pair of draws),
    returned as f32.  Element i depends only on (seed, offset + i)."""
    i = np.arange(offset, offset + n, dtype=np.uint64)
    a = splitmix64(seed, np.uint64(2) * i)
    b = splitmix64(seed, np.uint64(2) * i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32)


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (round-to-nearest-even; NaN stays a quiet NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r)
    return r.astype(np.uint16)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 to IEEE binary16 (numpy's cast is round-to-nearest-even)."""
    with np.errstate(over="ignore"):  # out-of-range values round to +-inf, as IEEE requires
        return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """simd.zig:123-126, via the C restatement."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().vtb_oracle_upcast_bf16(_ptr(bits), _ptr(out), bits.size)
    return out


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """forward.zig:661-666 (@floatCast f16 -> f32), via the C restatement."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().vtb_oracle_upcast_f16(_ptr(bits), _ptr(out), bits.size)
    return out


def to_dtype(x: np.ndarray, dtype: str):
    """Round f32 values to the storage dtype.  Returns (storage, exact_f32):
    storage is what the GPU holds (float32 or uint16 bit patterns) and
    exact_f32 is its exact upcast, the oracle's input."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f32":
        return x, x
    if dtype == "f16":
        b = f32_to_f16_bits(x)
        return b, f16_bits_to_f32(b)
    if dtype == "bf16":
        b = f32_to_bf16_bits(x)
        return b, bf16_bits_to_f32(b)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# Oracle calls
# ---------------------------------------------------------------------------
def softmax(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().vtb_oracle_softmax(_ptr(y), y.size)
    return y


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """math.rmsNorm (src/kernels/math.zig:11-32) of a copy of x."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    wf = np.ascontiguousarray(w, dtype=np.float32)
    lib().vtb_oracle_rmsnorm(_ptr(y), _ptr(wf), y.size, eps)
    return y


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """math.swiglu (math.zig:154-161): silu(gate) * up, as a new array."""
    g = np.ascontiguousarray(gate, dtype=np.float32).copy()
    u = np.ascontiguousarray(up, dtype=np.float32)
    lib().vtb_oracle_swiglu(_ptr(g), _ptr(u), g.size)
    return g


def geglu_approx(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """math.gegluApprox (math.zig:166-175), as a new array."""
    g = np.ascontiguousarray(gate, dtype=np.float32).copy()
    u = np.ascontiguousarray(up, dtype=np.float32)
    lib().vtb_oracle_geglu_approx(_ptr(g), _ptr(u), g.size)
    return g


def rope(x: np.ndarray, pos: int, base: float, half: bool = False) -> np.ndarray:
    """math.rope / math.ropeHalf (src/kernels/math.zig:85-133) applied to every
    head of x (shape [..., head_dim]); returns a rotated f32 copy."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    d = y.shape[-1]
    fn = lib().vtb_oracle_rope_half if half else lib().vtb_oracle_rope
    flat = y.reshape(-1, d)
    for h in range(flat.shape[0]):
        fn(flat.ctypes.data + h * d * 4, d, pos, base)
    return y


def rope_inv_freq(head_dim: int, base: float) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().vtb_oracle_rope_inv_freq(_ptr(out), head_dim, base)
    return out


QUANT_KINDS = {"q8_0": 0, "q4_k": 1, "q5_k": 2, "q6_k": 3}


def quant_block(kind: str):
    """(block_bytes, block_elems) of a GGUF block format (simd.zig)."""
    i = QUANT_KINDS[kind]
    return int(lib().vtb_oracle_quant_block_bytes(i)), int(lib().vtb_oracle_quant_block_elems(i))


def dequant(kind: str, blocks: np.ndarray) -> np.ndarray:
    """Dequantise whole blocks (uint8 bytes) to f32 (simd.zig dequantBlock*)."""
    bb, be = quant_block(kind)
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert b.size % bb == 0
    n = b.size // bb
    out = np.empty(n * be, np.float32)
    for i in range(n):
        lib().vtb_oracle_dequant_block(QUANT_KINDS[kind], b.ctypes.data + i * bb, out.ctypes.data + i * be * 4)
    return out


def matmul_quant(kind: str, w: np.ndarray, x: np.ndarray, m: int, k: int) -> np.ndarray:
    """out = W @ x for m rows of quantised weights (simd.zig matmul_*)."""
    wb = np.ascontiguousarray(w, dtype=np.uint8)
    xa = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(m, np.float32)
    rc = lib().vtb_oracle_matmul_quant(QUANT_KINDS[kind], _ptr(out), _ptr(wb), _ptr(xa), m, k)
    if rc != 0:
        raise ValueError("matmul_quant: k is not a whole number of blocks")
    return out


def matmul_batched(kind: str, w: np.ndarray, acts: np.ndarray, m: int, k: int, B: int) -> np.ndarray:
    """out[B, m]: dequantised weight rows . each token's activations
    (prefill.zig matmulBatched: dequantToF32 + simd.dot_f32)."""
    wb = np.ascontiguousarray(w, dtype=np.uint8)
    xa = np.ascontiguousarray(acts, dtype=np.float32).reshape(-1)
    assert xa.size == B * k
    out = np.empty(B * m, np.float32)
    rc = lib().vtb_oracle_matmul_batched(QUANT_KINDS[kind], _ptr(out), _ptr(wb), _ptr(xa), m, k, B)
    if rc != 0:
        raise ValueError("matmul_batched: k is not a whole number of blocks or above 32768")
    return out.reshape(B, m)


def argmax(x: np.ndarray) -> int:
    y = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().vtb_oracle_argmax(_ptr(y), y.size))


def window_start(pos: int, sliding_window: int = NO_WINDOW) -> int:
    return int(lib().vtb_oracle_window_start(pos, sliding_window))


class OracleKvCache:
    """kv_cache.zig:20-196 over numpy f32 storage (the oracle's view)."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq):
        total = n_layers * max_seq * n_kv_heads * head_dim
        self.k = np.zeros(total, np.float32)
        self.v = np.zeros(total, np.float32)
        self.c = KvCacheC(n_layers, n_kv_heads, head_dim, max_seq, _ptr(self.k), _ptr(self.v), 0)

    @property
    def pos(self):
        return self.c.pos

    @pos.setter
    def pos(self, p):
        self.c.pos = p

    @property
    def max_seq(self):
        return self.c.max_seq

    @property
    def row(self):
        return self.c.n_kv_heads * self.c.head_dim

    def key_slot(self, layer):
        off = lib().vtb_oracle_kv_slot_offset(ctypes.byref(self.c), layer)
        if off == NO_WINDOW:
            raise IndexError("slot out of range")
        return self.k[off:off + self.row]

    def value_slot(self, layer):
        off = lib().vtb_oracle_kv_slot_offset(ctypes.byref(self.c), layer)
        if off == NO_WINDOW:
            raise IndexError("slot out of range")
        return self.v[off:off + self.row]

    def keys_for(self, layer, n_tokens):
        off = lib().vtb_oracle_kv_layer_offset(ctypes.byref(self.c), layer)
        return self.k[off:off + n_tokens * self.row]

    def values_for(self, layer, n_tokens):
        off = lib().vtb_oracle_kv_layer_offset(ctypes.byref(self.c), layer)
        return self.v[off:off + n_tokens * self.row]

    def layer_rows(self, which, layer):
        """[max_seq, n_kv, head_dim] view of one layer of K or V."""
        arr = self.k if which == "k" else self.v
        n = self.c.max_seq * self.row
        off = layer * n
        return arr[off:off + n].reshape(self.c.max_seq, self.c.n_kv_heads, self.c.head_dim)

    def advance(self):
        if lib().vtb_oracle_kv_advance(ctypes.byref(self.c)) != 0:
            raise IndexError("KvCacheFull")

    def shrink_to_fit(self, new_max_seq):
        rc = lib().vtb_oracle_kv_shrink_to_fit(ctypes.byref(self.c), new_max_seq)
        if rc == 4:
            raise ValueError("NewMaxSeqBelowPos")


def config(n_heads, n_kv_heads, head_dim, max_seq, sliding_window=NO_WINDOW) -> ConfigC:
    return ConfigC(n_heads, n_kv_heads, head_dim, max_seq, sliding_window)


def cpu_attention(q: np.ndarray, cache: OracleKvCache, c: ConfigC, layer: int) -> np.ndarray:
    """forward.zig:187-228 for the query at cache.pos."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    scores = np.zeros(c.n_heads * c.max_seq, np.float32)
    out = np.zeros(c.n_heads * c.head_dim, np.float32)
    rc = lib().vtb_oracle_cpu_attention(_ptr(q), ctypes.byref(cache.c), ctypes.byref(c),
                                        layer, _ptr(scores), _ptr(out))
    if rc != 0:
        raise IndexError("cpu_attention: layer or pos out of range")
    return out


def attention_causal(q_all: np.ndarray, cache: OracleKvCache, c: ConfigC, layer: int,
                     rows) -> np.ndarray:
    """prefill.zig:237-287 for the listed batch positions b (query at
    cache.pos + b).  Returns [len(rows), n_heads*head_dim]."""
    q_all = np.ascontiguousarray(q_all, dtype=np.float32)
    qd = c.n_heads * c.head_dim
    B = q_all.size // qd
    scores = np.zeros(c.n_heads * c.max_seq, np.float32)
    full = np.zeros(B * qd, np.float32)
    for b in rows:
        rc = lib().vtb_oracle_attention_causal(_ptr(q_all), ctypes.byref(cache.c), ctypes.byref(c),
                                               layer, int(b), _ptr(scores), _ptr(full))
        if rc != 0:
            raise IndexError("attention_causal: out of range")
    return full.reshape(B, qd)[np.asarray(list(rows), dtype=np.int64)]


def attention_f64(q: np.ndarray, cache: OracleKvCache, c: ConfigC, layer: int, cur_pos: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(c.n_heads * c.head_dim, np.float64)
    rc = lib().vtb_oracle_attention_f64(_ptr(q), ctypes.byref(cache.c), ctypes.byref(c),
                                        layer, cur_pos, _ptr(out))
    if rc != 0:
        raise IndexError("attention_f64: out of range")
    return out


class Pool:
    """pool.zig ThreadPool restatement (CPU baseline only)."""

    def __init__(self, requested: int = 0):
        self.h = lib().vtb_oracle_pool_init(requested, os.cpu_count() or 1)

    @property
    def workers(self):
        return int(lib().vtb_oracle_pool_workers(self.h))

    def set_active(self, n):
        lib().vtb_oracle_pool_set_active(self.h, n)

    def sum(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a, dtype=np.uint32)
        return int(lib().vtb_oracle_pool_sum(self.h, _ptr(a), a.size))

    def attention(self, q, cache: OracleKvCache, c: ConfigC, layer: int, cur_pos: int, scores=None, out=None):
        q = np.ascontiguousarray(q, dtype=np.float32)
        if scores is None:
            scores = np.zeros(c.n_heads * c.max_seq, np.float32)
        if out is None:
            out = np.zeros(c.n_heads * c.head_dim, np.float32)
        rc = lib().vtb_oracle_cpu_attention_pooled(self.h, _ptr(q), ctypes.byref(cache.c), ctypes.byref(c),
                                                   layer, cur_pos, _ptr(scores), _ptr(out))
        if rc != 0:
            raise IndexError("pooled attention: out of range")
        return out

    def close(self):
        if self.h:
            lib().vtb_oracle_pool_deinit(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LayerWeights:
    """One decode layer's weights as the layer step uses them: f32 norm
    weights and GGUF-quantised projection blocks (raw bytes) of one kind."""

    def __init__(self, kind, attn_norm, wq, wk, wv, wo, ffn_norm, wgate, wup, wdown):
        self.kind = kind
        self.attn_norm, self.ffn_norm = attn_norm, ffn_norm
        self.wq, self.wk, self.wv, self.wo = wq, wk, wv, wo
        self.wgate, self.wup, self.wdown = wgate, wup, wdown


def cpu_layer_step(x: np.ndarray, lw: LayerWeights, cache: OracleKvCache, c: ConfigC, layer: int, dim: int,
                   ffn_dim: int, rms_eps: float, rope_base: float, rope_half: bool = False,
                   activation: str = "silu", kv_round=None) -> np.ndarray:
    """forward.cpuLayerStep (src/runtime/forward.zig:230-288) for one token at
    cache.pos, composed from the restatements above; returns the new x (f32)
    and writes this token's K/V rows into the cache slot.  kv_round, when
    given, maps the f32 K/V row to the values a lower-precision cache holds
    (the query stays f32, as State.q is)."""
    n_heads, n_kv, hd = c.n_heads, c.n_kv_heads, c.head_dim
    kv_dim = n_kv * hd
    xb = rms_norm(x, lw.attn_norm, rms_eps)
    q = matmul_quant(lw.kind, lw.wq, xb, dim, dim)
    k = matmul_quant(lw.kind, lw.wk, xb, kv_dim, dim)
    v = matmul_quant(lw.kind, lw.wv, xb, kv_dim, dim)
    q = rope(q.reshape(n_heads, hd), cache.pos, rope_base, rope_half).reshape(-1)
    k = rope(k.reshape(n_kv, hd), cache.pos, rope_base, rope_half).reshape(-1)
    if kv_round is not None:
        k, v = kv_round(k), kv_round(v)
    cache.key_slot(layer)[:] = k
    cache.value_slot(layer)[:] = v
    attn = cpu_attention(q, cache, c, layer)
    x = (x + matmul_quant(lw.kind, lw.wo, attn, dim, dim)).astype(np.float32)
    xb = rms_norm(x, lw.ffn_norm, rms_eps)
    gate = matmul_quant(lw.kind, lw.wgate, xb, ffn_dim, dim)
    up = matmul_quant(lw.kind, lw.wup, xb, ffn_dim, dim)
    h = swiglu(gate, up) if activation == "silu" else geglu_approx(gate, up)
    return (x + matmul_quant(lw.kind, lw.wdown, h, dim, ffn_dim)).astype(np.float32)


def cpu_prefill_layer(x: np.ndarray, lw: LayerWeights, cache: OracleKvCache, c: ConfigC, layer: int, dim: int,
                      ffn_dim: int, rms_eps: float, rope_base: float, rope_half: bool = False,
                      activation: str = "silu", kv_round=None) -> np.ndarray:
    """prefill.prefillLayer (src/runtime/prefill.zig:151-231) for the B tokens
    of x ([B][dim]) at positions cache.pos .. cache.pos+B-1; returns the new
    x and writes the B K/V rows into the cache.  kv_round, when given, maps
    the f32 K/V rows to the values a lower-precision cache holds, as the GPU
    path stores them; the queries stay f32, as the reference's s.q is
    (prefill.zig:167-197)."""
    B = x.shape[0]
    n_heads, n_kv, hd = c.n_heads, c.n_kv_heads, c.head_dim
    kv_dim = n_kv * hd
    pos0 = cache.pos
    xb = np.stack([rms_norm(x[b], lw.attn_norm, rms_eps) for b in range(B)])
    q = matmul_batched(lw.kind, lw.wq, xb, dim, dim, B).reshape(B, n_heads, hd)
    k = matmul_batched(lw.kind, lw.wk, xb, kv_dim, dim, B).reshape(B, n_kv, hd)
    v = matmul_batched(lw.kind, lw.wv, xb, kv_dim, dim, B).reshape(B, n_kv, hd)
    for b in range(B):
        q[b] = rope(q[b], pos0 + b, rope_base, rope_half)
        k[b] = rope(k[b], pos0 + b, rope_base, rope_half)
    if kv_round is not None:
        k, v = kv_round(k), kv_round(v)
    for b in range(B):
        cache.pos = pos0 + b
        cache.key_slot(layer)[:] = k[b].reshape(-1)
        cache.value_slot(layer)[:] = v[b].reshape(-1)
    cache.pos = pos0
    attn = attention_causal(q.reshape(B, -1), cache, c, layer, range(B))
    x = (x + matmul_batched(lw.kind, lw.wo, attn, dim, dim, B).reshape(B, dim)).astype(np.float32)
    xb = np.stack([rms_norm(x[b], lw.ffn_norm, rms_eps) for b in range(B)])
    gate = matmul_batched(lw.kind, lw.wgate, xb, ffn_dim, dim, B)
    up = matmul_batched(lw.kind, lw.wup, xb, ffn_dim, dim, B)
    h = (swiglu(gate, up) if activation == "silu" else geglu_approx(gate, up)).reshape(B, ffn_dim)
    return (x + matmul_batched(lw.kind, lw.wdown, h, dim, ffn_dim, B).reshape(B, dim)).astype(np.float32)

