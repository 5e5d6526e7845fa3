"""Checks on the built gfx950 code objects (vantablack_amd/_build/*.hsaco,
from __graft_entry__.build()), read from their AMDGPU metadata notes:
  - no kernel spills VGPRs or uses scratch (a spill to scratch is a silent
    slowdown the parity tests cannot see; the register allocator has
    produced them when kernel bodies were combined);
  - the LDS each DMA-staging kernel declares holds its stage arrays, and
    stays within the 160 KiB a gfx950 workgroup may hold.
Skipped when the code objects are not built here."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "vantablack_amd", "_build")
LLVM = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin")
FAMILIES = ("decode", "prefill", "gemv", "qgemm", "layer", "kvcopy")
LDS_MAX = 160 * 1024


def kernel_metadata(family, tmp_path):
    src = os.path.join(BUILD, f"{family}.hsaco")
    bundler, readelf = os.path.join(LLVM, "clang-offload-bundler"), os.path.join(LLVM, "llvm-readelf")
    if not (os.path.exists(src) and os.path.exists(bundler) and os.path.exists(readelf)):
        pytest.skip("code objects or LLVM tools not present")
    co = os.path.join(str(tmp_path), f"{family}.co")
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={src}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
    notes = subprocess.run([readelf, "--notes", co], check=True, capture_output=True, text=True).stdout
    kernels, cur = {}, {}
    for line in notes.splitlines():
        m = re.match(r"\s+\.(name|group_segment_fixed_size|private_segment_fixed_size|vgpr_spill_count|"
                     r"sgpr_spill_count):\s+(\S+)", line)
        if not m:
            continue
        cur[m.group(1)] = m.group(2)
        if {"name", "group_segment_fixed_size", "private_segment_fixed_size", "vgpr_spill_count"} <= cur.keys():
            kernels[cur["name"]] = {k: (v if k == "name" else int(v)) for k, v in cur.items()}
            cur = {}
    assert kernels, f"no kernel metadata in {family}.hsaco"
    return kernels


@pytest.mark.parametrize("family", FAMILIES)
def test_no_vgpr_spills_or_scratch(family, tmp_path):
    ks = kernel_metadata(family, tmp_path)
    bad = {n: (k["vgpr_spill_count"], k["private_segment_fixed_size"]) for n, k in ks.items()
           if k["vgpr_spill_count"] or k["private_segment_fixed_size"]}
    assert not bad, f"VGPR spills / scratch bytes per lane: {bad}"


@pytest.mark.parametrize("family", FAMILIES)
def test_lds_within_a_workgroup(family, tmp_path):
    for n, k in kernel_metadata(family, tmp_path).items():
        assert k["group_segment_fixed_size"] <= LDS_MAX, n


def test_prefill_lds_holds_the_dma_stages(tmp_path):
    ks = kernel_metadata("prefill", tmp_path)
    for d in (64, 128, 256):
        bn = 64 if d <= 128 else 32  # tiles.h prefill_block_n
        kbytes, vbytes = bn * (d // 8 + 1) * 16, d * (bn // 8 + 1) * 16  # PrefillLds<D>
        assert ks[f"vtb_prefill_d{d}"]["group_segment_fixed_size"] >= 2 * kbytes + 2 * vbytes


def test_mfma_decode_lds_holds_the_dma_stages(tmp_path):
    ks = kernel_metadata("decode", tmp_path)
    for kv in ("f16", "bf16"):
        for d in (64, 128, 256):
            for g in (4, 8, 16):
                if g >= 16 and d >= 256:
                    continue  # scalar form (tiles.h decode_uses_mfma)
                nw = (4 if d >= 256 else 8) // (2 if g >= 16 else 1)
                sb = 2 * 16 * 2 * d  # bytes per wave per stage
                assert ks[f"vtb_decode_{kv}_d{d}_g{g}"]["group_segment_fixed_size"] >= 2 * nw * sb
