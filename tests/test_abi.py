"""CPU-only checks of the C-ABI library: it is built, loads, exports every
symbol include/vtb_hip.h declares (and nothing in Python binds a symbol the
header lacks), and its host logic rejects bad handles without a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vtb_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(vtb_hip_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def hip():
    from vantablack_amd import hip
    return hip


def test_library_exports_every_declared_symbol(hip):
    L = hip.lib()
    syms = declared_symbols()
    assert len(syms) >= 30
    for s in sorted(syms):
        assert hasattr(L, s), f"{s} declared in vtb_hip.h but not exported"
    assert set(hip.SIGNATURES) == syms


def test_null_handles_are_rejected_without_a_gpu(hip):
    L = hip.lib()
    assert L.vtb_hip_wait_idle(None) == hip.EINVAL
    assert not L.vtb_hip_segment_begin(None)
    assert L.vtb_hip_segment_commit(None) == hip.EINVAL
    assert L.vtb_hip_kv_cache_pos(None) == 0
    assert L.vtb_hip_kv_cache_advance(None) == hip.EINVAL
    assert L.vtb_hip_kv_cache_slot_offset(None, 0) == (1 << 64) - 1
    assert L.vtb_hip_kv_cache_shrink_to_fit(None, 1) == hip.EINVAL
    assert not L.vtb_hip_alloc(None, 16)
    assert not L.vtb_hip_kv_cache_init(None, 1, 1, 64, 1, 0)
    assert L.vtb_hip_last_error(None) == b""
    assert L.vtb_hip_stream(None) is None
    cfg = hip.AttnConfigC(8, 8, 64, 16, hip.NO_WINDOW)
    assert L.vtb_hip_layer_attention(None, None, ctypes.byref(cfg), 0, None, None, None, None) == hip.EINVAL
    assert L.vtb_hip_reserve(None, ctypes.byref(cfg), 0, 16, 0, 0.0) == hip.EINVAL
    assert L.vtb_hip_scratch_bytes(None) == 0


def test_code_objects_are_gfx950(hip):
    data = open(hip.LIB_PATH, "rb").read()
    assert data.count(b"amdgcn-amd-amdhsa--gfx950") >= 3
