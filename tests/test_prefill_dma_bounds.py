"""CPU-side bounds model of the prefill kernel's tile DMA (TileDma in
vantablack_amd/csrc/kernels/prefill.hip; the launcher's limits in
launch_prefill_mfma, vantablack_amd/csrc/vtb_hip.cpp).

The model enumerates, for every wave, block and lane, the LDS bytes each
`buffer_load_dwordx4 ... lds` writes and the buffer offset it reads, with the
kernel's own tile constants, and checks:
  - every LDS write lies inside its stage array, and every slot of the padded
    stage layout is written exactly once per tile;
  - every K read of a row before the block's last key lies wholly inside the
    tile's buffer descriptor and inside the key allocation; every read of a
    later row lies wholly past the descriptor's range (the hardware range
    check returns zero without a memory access);
  - every V^T read lies inside its descriptor and inside the head's V^T
    allocation;
  - offsets and descriptor sizes fit the 32-bit fields at the largest prompt
    the launcher accepts.
"""
import itertools

import pytest

NW = 4  # waves per workgroup (VTB_PREFILL: __launch_bounds__(256, ...), prefill_entry<D, 4>)


def block_n(d):  # tiles.h prefill_block_n
    return 64 if d <= 128 else 32


def tile_dma_model(d):
    bn = block_n(d)
    kch, vch = d // 8, bn // 8
    ksl, vsl = bn * (kch + 1), d * (vch + 1)
    kbl, vbl = -(-ksl // 64), -(-vsl // 64)
    kpw, vpw = -(-kbl // NW), -(-vbl // NW)
    return dict(bn=bn, kch=kch, vch=vch, ksl=ksl, vsl=vsl, kbl=kbl, vbl=vbl, kpw=kpw, vpw=vpw)


def dma_lanes(m, which):
    """(wave, blk, lane, slot, row, chunk_read) for every active DMA lane."""
    ch_per_row = (m["kch"] if which == "k" else m["vch"]) + 1
    nsl, nbl, npw = (m["ksl"], m["kbl"], m["kpw"]) if which == "k" else (m["vsl"], m["vbl"], m["vpw"])
    for wave in range(NW):
        for i in range(npw):
            blk = wave + NW * i
            if blk >= nbl:
                continue
            for lane in range(64):
                s = 64 * blk + lane
                if nsl % 64 != 0 and s >= nsl:
                    continue
                row, ch = divmod(s, ch_per_row)
                yield wave, blk, lane, s, row, (0 if ch == ch_per_row - 1 else ch)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_lds_writes_stay_in_stage_and_cover_it(d):
    m = tile_dma_model(d)
    for which, nsl in (("k", m["ksl"]), ("v", m["vsl"])):
        stage_bytes = nsl * 16  # PrefillLds<D>::KBYTES / VBYTES
        seen = [0] * nsl
        for wave, blk, lane, s, row, ch in dma_lanes(m, which):
            lo = 1024 * blk + 16 * lane
            assert 0 <= lo and lo + 16 <= stage_bytes, (which, d, wave, blk, lane)
            assert lo == 16 * s
            seen[s] += 1
        assert all(c == 1 for c in seen), (which, d)


@pytest.mark.parametrize("d,n_kv,layout", [(64, 8, "f16"), (128, 8, "f16"), (128, 1, "f16"), (256, 1, "f16"),
                                           (64, 1, "bf16"), (128, 1, "bf16"), (256, 1, "bf16")])
def test_k_reads_in_range_or_wholly_past_it(d, n_kv, layout):
    m = tile_dma_model(d)
    bn = m["bn"]
    # f16 caches are read in place ([row][n_kv][D]); bf16 caches through the
    # conversion pass's f16 keys ([n_kv][vt_ld][D]).
    krow = 2 * (n_kv * d if layout == "f16" else d)
    for n_rows in (1, 5, bn - 1, bn, bn + 3, 3 * bn, 3 * bn + 17):
        kend = n_rows  # keys [0, kend) exist (the block's last key + 1)
        for kt0 in range(0, kend, bn):
            rows = min(kend - kt0, bn)
            num_records = rows * krow
            assert num_records < 2 ** 32
            for wave, blk, lane, s, row, ch in dma_lanes(m, "k"):
                off = row * krow + 16 * ch
                assert off < 2 ** 31
                if row < rows:
                    assert off + 16 <= num_records
                    assert kt0 * krow + off + 16 <= kend * krow  # inside the existing keys
                else:
                    assert off >= num_records  # range check: zero, no access


@pytest.mark.parametrize("d", [64, 128, 256])
def test_v_reads_in_range(d):
    m = tile_dma_model(d)
    bn = m["bn"]
    for vt_ld in (64, 128, 64 * 37):
        vrow = 2 * vt_ld
        num_records = (d - 1) * vrow + bn * 2
        for kt0 in range(0, vt_ld, bn):
            for wave, blk, lane, s, row, ch in dma_lanes(m, "v"):
                off = row * vrow + 16 * ch
                assert off + 16 <= num_records
                assert 2 * kt0 + off + 16 <= d * vt_ld * 2  # inside the head's V^T


@pytest.mark.parametrize("d,n_kv", itertools.product([64, 128, 256], [1, 8, 64]))
def test_launcher_limits_keep_offsets_32_bit(d, n_kv):
    # launch_prefill_mfma refuses vt_ld with head_dim * vt_ld * 2 >= 2^31 or
    # n_kv * head_dim * 2 * bn >= 2^31; at the largest accepted values the
    # kernel's int offsets and u32 descriptor sizes still fit.
    m = tile_dma_model(d)
    bn = m["bn"]
    vt_ld = ((2 ** 31 - 1) // (2 * d)) // 64 * 64
    assert d * vt_ld * 2 < 2 ** 31
    vrow = 2 * vt_ld
    assert (d - 1) * vrow + bn * 2 < 2 ** 31
    assert max(row * vrow + 16 * ch for _, _, _, _, row, ch in dma_lanes(m, "v")) < 2 ** 31
    krow = 2 * n_kv * d
    if n_kv * d * 2 * bn < 2 ** 31:
        assert max(row * krow + 16 * ch for _, _, _, _, row, ch in dma_lanes(m, "k")) < 2 ** 31
        assert bn * krow < 2 ** 32


def _k_tile_accesses(m, krow, kend, kt0, pad_chunk, clamp):
    """Memory bytes [lo, hi) relative to the key allocation's start that the K
    DMA of the tile at kt0 touches, for an addressing variant: the pad slot
    reads chunk 0 of its row (pad_chunk 0, the current kernel) or another
    chunk (KCH: one chunk past the row's D elements); the descriptor covers
    the rows before kend (clamp, the current kernel) or all BN rows of the
    tile.  Accesses the range check drops (offset + 16 > num_records) touch
    nothing."""
    rows = min(kend - kt0, m["bn"]) if clamp else m["bn"]
    num_records = rows * krow
    ch_per_row = m["kch"] + 1
    res = []
    for _, _, _, s, row, _ in dma_lanes(m, "k"):
        ch = s % ch_per_row
        off = row * krow + 16 * (pad_chunk if ch == m["kch"] else ch)
        if off + 16 <= num_records:
            res.append((kt0 * krow + off, kt0 * krow + off + 16))
    return res


@pytest.mark.parametrize("pad_chunk,clamp,inside", [
    (0, True, True),     # the current kernel: pad slots read chunk 0, descriptor ends at kend
    ("KCH", True, True),  # pad slots one chunk past the row: range-checked (or inside the allocation)
    (0, False, False),   # descriptor over all BN rows: reads rows past kend, outside a kend-row buffer
])
def test_addressing_variants_on_a_48_key_buffer(pad_chunk, clamp, inside):
    # The 48-token d128 case that faulted an earlier direct-to-LDS version,
    # with K read in place from an f16 cache holding exactly 48 rows of one KV
    # head (krow = 2 D bytes): which addressing variants touch memory outside
    # the allocation [0, 48 krow)?  The pad-slot offset alone cannot (the
    # range check drops whatever passes the descriptor); a descriptor that is
    # not clamped to the existing keys does.
    d, n_rows = 128, 48
    m = tile_dma_model(d)
    krow = 2 * d
    pc = m["kch"] if pad_chunk == "KCH" else pad_chunk
    acc = []
    for kt0 in range(0, n_rows, m["bn"]):
        acc += _k_tile_accesses(m, krow, n_rows, kt0, pc, clamp)
    outside = [a for a in acc if a[0] < 0 or a[1] > n_rows * krow]
    assert (not outside) == inside, outside[:4]


def test_stage_arrays_and_lds_pointers():
    # The four stage arrays are separate __shared__ objects of exactly the
    # modelled sizes (so a write inside a stage is inside the workgroup's
    # allocation; test_code_objects checks that allocation holds them), and
    # every DMA destination is an LDS-address-space pointer derived from
    # them: M0 comes from a local (32-bit LDS) address, never from a generic
    # pointer converted at run time.
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = open(os.path.join(root, "vantablack_amd", "csrc", "kernels", "prefill.hip")).read()
    for decl in ("__shared__ __attribute__((aligned(16))) char s_k0[PrefillLds<D>::KBYTES];",
                 "__shared__ __attribute__((aligned(16))) char s_k1[PrefillLds<D>::KBYTES];",
                 "__shared__ __attribute__((aligned(16))) char s_v0[PrefillLds<D>::VBYTES];",
                 "__shared__ __attribute__((aligned(16))) char s_v1[PrefillLds<D>::VBYTES];",
                 # the key-split form's second tile of each step: the same sizes
                 "__shared__ __attribute__((aligned(16))) char s_k2[KSPLIT ? PrefillLds<D>::KBYTES : 16];",
                 "__shared__ __attribute__((aligned(16))) char s_k3[KSPLIT ? PrefillLds<D>::KBYTES : 16];",
                 "__shared__ __attribute__((aligned(16))) char s_v2[KSPLIT ? PrefillLds<D>::VBYTES : 16];",
                 "__shared__ __attribute__((aligned(16))) char s_v3[KSPLIT ? PrefillLds<D>::VBYTES : 16];",
                 "PrefillLds<D> lds{(lchar*)s_k0, (lchar*)s_k1, (lchar*)s_v0, (lchar*)s_v1,\n"
                 "                    (lchar*)s_k2, (lchar*)s_k3, (lchar*)s_v2, (lchar*)s_v3};",
                 # a second-half tile is fetched only below the item's last key
                 "if (t + BN < ikend) fetch(t + BN, kb, vb);",
                 "static constexpr int KBYTES = BN * (D / 8 + 1) * 16;",
                 "static constexpr int VBYTES = D * (BN / 8 + 1) * 16;",
                 "typedef __attribute__((address_space(3))) char lchar;"):
        assert decl in src, decl
    for d in (64, 128, 256):
        m = tile_dma_model(d)
        assert m["ksl"] * 16 == m["bn"] * (d // 8 + 1) * 16  # KBYTES
        assert m["vsl"] * 16 == d * (m["bn"] // 8 + 1) * 16  # VBYTES
    # Every buffer-to-LDS DMA in the kernels takes an address_space(3)
    # destination built from an lchar / dchar stage pointer.
    import re
    for name in ("prefill.hip", "decode.hip"):
        text = open(os.path.join(root, "vantablack_amd", "csrc", "kernels", name)).read()
        calls = [m.start() for m in re.finditer(r"__builtin_amdgcn_raw_ptr_buffer_load_lds\(", text)]
        assert calls, name
        for c in calls:
            args = text[c:text.index(";", c)]
            assert "address_space(3)" in args, (name, args)


def test_model_constants_match_the_sources():
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    tiles = open(os.path.join(root, "vantablack_amd", "csrc", "tiles.h")).read()
    assert "prefill_block_n(int head_dim) { return head_dim <= 128 ? 64 : 32; }" in tiles
    src = open(os.path.join(root, "vantablack_amd", "csrc", "kernels", "prefill.hip")).read()
    assert "vtb::prefill_entry<D, 4>(a);" in src
    for expr in ("static constexpr int KSL = BN * (KCH + 1);", "static constexpr int VSL = D * (VCH + 1);",
                 "const int sl = 64 * (wave + NW * i) + lane, row = sl / (KCH + 1), ch = sl % (KCH + 1);",
                 "koff[i] = row * krow_bytes + 16 * (ch == KCH ? 0 : ch);",
                 "voff[i] = row * vrow_bytes + 16 * (ch == VCH ? 0 : ch);",
                 "(kl + 1024 * blk)", "(vl + 1024 * blk)"):
        assert expr in src, expr
