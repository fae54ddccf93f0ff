"""MI355X-native paged KV-cache hot path of IVA1.0.

Host side in Python on PyTorch-ROCm (tensors, streams, the page allocator);
compute in hand-written gfx950 HIP kernels behind the C ABI of
include/ivakv.h (libivakv.so, bound with ctypes in ``_abi``).

The directory name is not a Python identifier; load it with
``__graft_entry__.load_package()``, which registers it as ``iva_amd``.
"""
from . import _abi, model, paged_cache, workloads
from .ops import (
    chunk_elems,
    copy_pages,
    decode_workspace_bytes,
    dtype_code,
    is_fp8,
    kv_append,
    kv_compact,
    kv_gather,
    kv_ops,
    KVOps,
    paged_decode_append_attention,
    paged_decode_attention,
    paged_decode_attention_merge,
    paged_decode_attention_partial,
    paged_prefill_attention,
    prefill_split_workspace_bytes,
    pool_geometry,
    pool_shapes,
    rope_,
    scale_shape,
)
from .model import PagedAttention, Transformer, TransformerConfig, get_attention
from .paged_cache import OutOfPagesError, PagedKVCache, PagedKVPool, create_kv_cache

__all__ = [
    "OutOfPagesError",
    "PagedAttention",
    "PagedKVCache",
    "PagedKVPool",
    "Transformer",
    "TransformerConfig",
    "create_kv_cache",
    "get_attention",
    "chunk_elems",
    "copy_pages",
    "decode_workspace_bytes",
    "dtype_code",
    "is_fp8",
    "kv_append",
    "kv_compact",
    "kv_gather",
    "kv_ops",
    "KVOps",
    "paged_decode_append_attention",
    "paged_decode_attention",
    "paged_decode_attention_merge",
    "paged_decode_attention_partial",
    "paged_prefill_attention",
    "prefill_split_workspace_bytes",
    "pool_geometry",
    "pool_shapes",
    "rope_",
    "scale_shape",
]
