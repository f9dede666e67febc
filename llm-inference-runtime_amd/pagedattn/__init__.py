"""MI355X (gfx950) paged attention for the mini-vLLM serving engine.

``import pagedattn as flashinfer`` gives the engine's attention shim the
FlashInfer entry points it uses; ``pagedattn.llama`` is a drop-in for the
shim itself (src/models/llama.py).  All compute runs in libpagedattn.so;
nothing here falls back to PyTorch.
"""

from .ops import (  # noqa: F401
    PAGE_SIZE,
    BatchDecodeWithPagedKVCacheWrapper,
    BatchPrefillWithPagedKVCacheWrapper,
    append_paged_kv_cache,
    append_paged_kv_cache_e4m3_amax,
    apply_rope_pos_ids_inplace,
    build_paged_metadata,
    copy_bytes,
    fork_pages,
    get_batch_indices_positions,
    quantize_pages_e4m3,
    read_bytes,
    rope_append_paged_kv_cache,
)
from ._lib import LIB_PATH, PagedAttnError, lib  # noqa: F401

__all__ = [
    "PAGE_SIZE",
    "BatchDecodeWithPagedKVCacheWrapper",
    "BatchPrefillWithPagedKVCacheWrapper",
    "append_paged_kv_cache",
    "append_paged_kv_cache_e4m3_amax",
    "apply_rope_pos_ids_inplace",
    "build_paged_metadata",
    "copy_bytes",
    "fork_pages",
    "get_batch_indices_positions",
    "quantize_pages_e4m3",
    "read_bytes",
    "rope_append_paged_kv_cache",
    "LIB_PATH",
    "PagedAttnError",
    "lib",
]
