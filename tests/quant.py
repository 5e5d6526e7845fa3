"""Quantised-weight fixtures for the GEMV tests (random bytes with finite f16
super-scales, the construction of bridge.zig:362-376 fixupKQuantScales, with
Q8_0 given the same treatment) and an independent vectorised numpy
dequantiser used to pin the C oracle."""
import numpy as np

BLOCK = {"q8_0": (34, 32), "q4_k": (144, 256), "q5_k": (176, 256), "q6_k": (210, 256)}


def _f16(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def random_weights(kind, m, k, seed):
    """m rows of k weights in `kind`'s block format, as uint8 bytes."""
    bb, be = BLOCK[kind]
    assert k % be == 0
    rng = np.random.default_rng(seed)
    nblk = m * (k // be)
    w = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    d = _f16(0.001 + rng.random(nblk) * 0.05)
    if kind == "q8_0":
        w[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    elif kind in ("q4_k", "q5_k"):
        w[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
        w[:, 2:4] = _f16(rng.random(nblk) * 0.05).view(np.uint8).reshape(nblk, 2)
    else:
        w[:, 208:210] = d.view(np.uint8).reshape(nblk, 2)
    return w.reshape(-1)


def _f16_at(b, off):
    return b[:, off:off + 2].copy().view(np.float16).astype(np.float32).reshape(-1)


def np_dequant(kind, blocks):
    """Vectorised restatement of simd.zig's dequantBlock* for n blocks."""
    bb, be = BLOCK[kind]
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1, bb)
    n = b.shape[0]
    if kind == "q8_0":
        return (_f16_at(b, 0)[:, None] * b[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
    if kind in ("q4_k", "q5_k"):
        d, dmin = _f16_at(b, 0), _f16_at(b, 2)
        sc_b = b[:, 4:16].astype(np.uint32)
        sc = np.empty((n, 8), np.uint32)
        mn = np.empty((n, 8), np.uint32)
        sc[:, :4] = sc_b[:, 0:4] & 0x3F
        mn[:, :4] = sc_b[:, 4:8] & 0x3F
        sc[:, 4:] = (sc_b[:, 8:12] & 0x0F) | ((sc_b[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (sc_b[:, 8:12] >> 4) | ((sc_b[:, 4:8] >> 6) << 4)
        qs = b[:, 48:176] if kind == "q5_k" else b[:, 16:144]
        qs = qs.reshape(n, 4, 32).astype(np.uint32)
        q = np.empty((n, 8, 32), np.uint32)
        q[:, 0::2, :] = qs & 0x0F
        q[:, 1::2, :] = qs >> 4
        if kind == "q5_k":
            qh = b[:, 16:48].astype(np.uint32)           # [n, 32]
            bits = (qh[:, None, :] >> np.arange(8, dtype=np.uint32)[None, :, None]) & 1
            q = q + 16 * bits
        d1 = (d[:, None] * sc.astype(np.float32))          # f32 products, as the reference
        m1 = (dmin[:, None] * mn.astype(np.float32))
        w = d1[:, :, None] * q.astype(np.float32) - m1[:, :, None]
        return w.astype(np.float32).reshape(-1)
    # q6_k
    d = _f16_at(b, 208)
    ql = b[:, 0:128].reshape(n, 2, 64).astype(np.int32)
    qh = b[:, 128:192].reshape(n, 2, 32).astype(np.int32)
    sc = b[:, 192:208].view(np.int8).reshape(n, 2, 8).astype(np.float32)
    lo, hi = ql[:, :, :32], ql[:, :, 32:]
    q = np.stack([(lo & 0x0F) | (((qh >> 0) & 3) << 4), (hi & 0x0F) | (((qh >> 2) & 3) << 4),
                  (lo >> 4) | (((qh >> 4) & 3) << 4), (hi >> 4) | (((qh >> 6) & 3) << 4)], axis=2) - 32
    # q: [n, half, quadrant, l]; scale index is l//16 + 2*quadrant
    is_ = (np.arange(32) // 16)[None, None, None, :] + 2 * np.arange(4)[None, None, :, None]
    s = np.take_along_axis(sc[:, :, None, :].repeat(4, axis=2), np.broadcast_to(is_, (n, 2, 4, 32)), axis=3)
    w = (d[:, None, None, None] * s) * q.astype(np.float32)
    return w.astype(np.float32).reshape(-1)
