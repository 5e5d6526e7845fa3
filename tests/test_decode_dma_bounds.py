"""CPU-side bounds model of the MFMA decode kernel's tile DMA
(decode_mfma_body in vantablack_amd/csrc/kernels/decode.hip; the launcher's
row-width limit in vantablack_amd/csrc/vtb_hip.cpp).

Each wave stages 16-row blocks of K and V of one KV head in its own region
of two LDS stage arrays (s_stg0, s_stg1; NW * SB bytes each).  Block j's NI
instructions per operand write 64 lanes x 16 bytes from M0 = the wave's
region + 1024 i (+ VOFF for V), and lane l of instruction i reads chunk
(s % C) ^ swizzle(row) of row s / C, s = 64 i + l, through a raw buffer
descriptor over the block's nr rows.  The model enumerates every wave,
instruction and lane with the kernel's own constants and checks:
  - every LDS write lies inside the wave's region of its stage array, K in
    the first 16 rows' bytes and V after VOFF, and every slot of the region
    is written exactly once per block;
  - the chunk read is a permutation of the row's chunks, so the staged block
    holds every (row, chunk) exactly once;
  - reads of rows before nr lie inside the descriptor and inside the KV
    head's own D elements of that cache row; reads of rows at or past nr lie
    wholly past the descriptor (the hardware range check returns zero
    without a memory access);
  - offsets and descriptor sizes fit their 32-bit fields for every
    n_kv * D the launcher accepts;
  - a wave's f32 partial (G x D) fits the stage region it is written to.
"""
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "vantablack_amd", "csrc", "kernels", "decode.hip")
TILES = os.path.join(ROOT, "vantablack_amd", "csrc", "tiles.h")
HOST = os.path.join(ROOT, "vantablack_amd", "csrc", "vtb_hip.cpp")


def mfma_waves(d, g):  # tiles.h decode_mfma_waves (VTB_DECODE_MFMA_WAVES 8, _D256 8)
    return 8 // (2 if g >= 16 else 1)


def mfma_stages(d):  # tiles.h decode_mfma_stages (VTB_DECODE_MFMA_STAGES_D256 1)
    return 1 if d >= 256 else 2


def kswz(d, r):
    return r % (d // 8)


def vswz(d, r):
    return (2 * r) % (d // 8)


def model(d, g):
    C = d // 8
    RB = 2 * d
    VOFF = 16 * RB
    SB = 2 * 16 * RB
    NI = 16 * C // 64
    return dict(C=C, RB=RB, VOFF=VOFF, SB=SB, NI=NI, NW=mfma_waves(d, g))


# The MFMA form's shapes (tiles.h decode_uses_mfma: groups of 9-16 at d256
# take the scalar form).
SHAPES = [(d, g) for d in (64, 128, 256) for g in (4, 8, 16) if not (g >= 16 and d >= 256)]


@pytest.mark.parametrize("d,g", SHAPES)
def test_lds_writes_stay_in_the_waves_region_and_cover_it(d, g):
    m = model(d, g)
    assert m["NI"] * 64 == 16 * m["C"] and m["NI"] >= 1
    for stage in range(mfma_stages(d)):
        array_bytes = m["NW"] * m["SB"]  # s_stg0 / s_stg1
        seen = [0] * array_bytes
        for wave in range(m["NW"]):
            region = wave * m["SB"]
            for base in (0, m["VOFF"]):
                for i in range(m["NI"]):
                    m0 = region + base + 1024 * i
                    for lane in range(64):
                        lo = m0 + 16 * lane
                        assert region + base <= lo and lo + 16 <= region + base + 16 * m["RB"]
                        assert lo + 16 <= array_bytes
                        for b in range(lo, lo + 16):
                            seen[b] += 1
        assert all(c == 1 for c in seen), (d, g, stage)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_swizzled_reads_cover_each_row_once(d):
    m = model(d, 4)
    for swz in (kswz, vswz):
        got = set()
        for i in range(m["NI"]):
            for lane in range(64):
                s = 64 * i + lane
                r, cs = divmod(s, m["C"])
                ch = cs ^ swz(d, r)
                assert 0 <= ch < m["C"]
                got.add((r, ch))
        assert got == {(r, c) for r in range(16) for c in range(m["C"])}


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("n_kv", [1, 2, 8, 32])
def test_source_reads_in_the_head_or_past_the_descriptor(d, n_kv):
    m = model(d, 4)
    rs = n_kv * d * 2  # cache row stride, bytes
    for kvh in {0, n_kv - 1}:
        head_lo, head_hi = kvh * d * 2, (kvh + 1) * d * 2  # the head's bytes within a row
        for nr in range(1, 17):  # rows in the block (the last block of a wave may be short)
            num_records = nr * rs
            assert num_records < 2 ** 32
            for swz in (kswz, vswz):
                for i in range(m["NI"]):
                    for lane in range(64):
                        s = 64 * i + lane
                        r, cs = divmod(s, m["C"])
                        off = r * rs + 16 * (cs ^ swz(d, r))
                        if r < nr:
                            assert off + 16 <= num_records
                            within = head_lo + (off - r * rs)  # relative to the row's start
                            assert head_lo <= within and within + 16 <= head_hi
                        else:
                            assert off >= num_records


@pytest.mark.parametrize("d", [64, 128, 256])
def test_launcher_row_limit_keeps_offsets_32_bit(d):
    # vtb_hip.cpp refuses n_kv * D * 2 * 16 >= 2^31 for the MFMA form; at the
    # largest accepted n_kv the per-lane offsets (rows 0..15) and the
    # descriptor size still fit a signed 32-bit int.
    m = model(d, 4)
    n_kv = ((2 ** 31 - 1) // (d * 2 * 16))
    assert n_kv * d * 2 * 16 < 2 ** 31
    rs = n_kv * d * 2
    top = max(r * rs + 16 * ((cs ^ kswz(d, r)) | (cs ^ vswz(d, r)))
              for r in range(16) for cs in range(m["C"]))
    assert top + 16 < 2 ** 31
    assert 16 * rs < 2 ** 31


@pytest.mark.parametrize("d,g", SHAPES)
def test_partial_fits_its_stage_region(d, g):
    m = model(d, g)
    assert g * d * 4 <= m["SB"]


def test_model_constants_match_the_sources():
    src = open(SRC).read()
    for expr in ("constexpr int C = D / 8;", "constexpr int RB = 2 * D;", "constexpr int VOFF = 16 * RB;",
                 "constexpr int SB = 2 * 16 * RB;", "constexpr int NI = 16 * C / 64;",
                 "__shared__ __attribute__((aligned(16))) char s_stg0[NW * SB];",
                 "constexpr int NSTG = decode_mfma_stages(D);",
                 "__shared__ __attribute__((aligned(16))) char s_stg1[NSTG > 1 ? NW * SB : 16];",
                 "dchar* const stg1 = (dchar*)s_stg1 + (NSTG > 1 ? wave * SB : 0);",
                 "if (NSTG > 1 && n_blk > 1) issue(1, stg1);",
                 "const int s = 64 * i + lane, r = s / C, cs = s % C;",
                 "koff[i] = (int)(r * rs) + 16 * (cs ^ kswz<D>(r));",
                 "voff[i] = (int)(r * rs) + 16 * (cs ^ vswz<D>(r));",
                 "dchar* const stg0 = (dchar*)s_stg0 + wave * SB;",
                 "const long long nr = w1 - t0 < 16 ? w1 - t0 : 16;",
                 "const auto rk = buffer_rsrc(kbase + t0 * rs, (unsigned)(nr * rs));",
                 "const auto rv = buffer_rsrc(vbase + t0 * rs, (unsigned)(nr * rs));",
                 "(st + 1024 * i), 16,", "(st + VOFF + 1024 * i),",
                 "__device__ constexpr int kswz(int r) { return r % (D / 8); }",
                 "__device__ constexpr int vswz(int r) { return (2 * r) % (D / 8); }",
                 "typedef __attribute__((address_space(3))) char dchar;"):
        assert expr in src, expr
    tiles = open(TILES).read()
    assert "return (head_dim >= 256 ? VTB_DECODE_MFMA_WAVES_D256 : VTB_DECODE_MFMA_WAVES) / (g >= 16 ? 2 : 1);" \
        in tiles
    assert "#define VTB_DECODE_MFMA_WAVES 8" in tiles and "#define VTB_DECODE_MFMA_WAVES_D256 8" in tiles
    assert "#define VTB_DECODE_MFMA_STAGES_D256 1" in tiles
    assert ("constexpr int decode_mfma_stages(int head_dim) { return head_dim >= 256 ? "
            "VTB_DECODE_MFMA_STAGES_D256 : 2; }") in tiles
    assert "return kv_bytes == 2 && g >= 4 && !(g >= 16 && head_dim >= 256);" in tiles
    host = open(HOST).read()
    assert "(long long)(n_kv * head_dim) * 2 * 16 >= (1LL << 31)" in host
