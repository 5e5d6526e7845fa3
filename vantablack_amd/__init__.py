"""vantablack_amd: MI355X-native (gfx950) KV-cache attention for vantablack.

The product is the C-ABI library libvtb_hip.so (include/vtb_hip.h) built from
vantablack_amd/csrc; `vantablack_amd.hip` is its host-side mirror of
vantablack's attention interface.  Build with `python -m vantablack_amd.build`.
"""
from . import hip  # noqa: F401
from .hip import (  # noqa: F401
    BF16, F16, F32, NO_WINDOW, Buffer, Context, HipAttentionBackend, HipError, KvCache,
    KvCacheFull, LlamaConfig, NewMaxSeqBelowPos, Segment, layer_attention, layer_attention_rope,
    prefill_attention,
    step_attention,
)
