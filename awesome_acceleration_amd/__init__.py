"""MI355X-native (gfx950) attention hot path for the Qwen3 serving engine.

Drop-in replacements for the reference engine's ``flash_attn`` calls and its
``index_copy_`` KV store, implemented by hand-written HIP kernels in
``libaac_attn.so`` (C ABI: include/aac_attn.h).
"""
from .flash_attn_interface import (  # noqa: F401
    decode_paged,
    flash_attn_func,
    flash_attn_varlen_func,
    flash_attn_with_kvcache,
    kv_store,
    varlen_prefill_with_kvcache,
)
from .paged import BlockAllocator, SlotCacheManager  # noqa: F401

__version__ = "0.1.0"
