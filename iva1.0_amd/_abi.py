"""ctypes binding of libivakv.so (declarations in include/ivakv.h).

This is the whole Python <-> native boundary: plain pointers, sizes and a
stream handle go in, an int status comes out.  A non-zero status is raised as
:class:`IvakvError` carrying the library's thread-local message.

The library is loaded from ``$IVAKV_LIB`` or from ``libivakv.so`` next to this
file (built by ``build.py``).  If it is missing, :func:`lib` raises: there is no
fallback implementation behind these entry points.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, POINTER
from pathlib import Path
from typing import Optional

ABI_VERSION = 2

OK = 0
E_ARG = -1
E_DTYPE = -2
E_SHAPE = -3
E_LAUNCH = -4
E_WORKSPACE = -5

F32 = 0
F16 = 1
BF16 = 2

_I32P = POINTER(ctypes.c_int32)
_I64P = POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/ivakv.h one for one.
_DECODE_ARGS = [
    c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
    c_void_p, c_void_p,                    # block_tables, context_lens
    c_void_p, c_void_p, c_size_t,          # out, workspace, workspace_bytes
    c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
    c_int, c_int, c_int, c_float,          # block_size, max_blocks, num_pages, scale
    c_int, c_int, c_int, c_int,            # window, n_sink, partition_pages, dtype
    c_void_p,                              # stream
]

SIGNATURES = {
    "ivakv_abi_version": (c_int, []),
    "ivakv_last_error": (ctypes.c_char_p, []),
    "ivakv_append": (c_int, [
        c_void_p, c_void_p,                # k_new, v_new
        c_int64, c_int64, c_int64, c_int64,  # k tok/head strides, v tok/head strides
        c_void_p, c_void_p, c_void_p,      # k_pool, v_pool, slot_mapping
        c_int, c_int, c_int, c_int, c_int, c_int,  # n_tok, Hkv, D, block_size, num_pages, dtype
        c_void_p,                          # stream
    ]),
    "ivakv_gather": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, block_tables, context_lens
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,  # B, max_blocks, Hkv, D, bs, num_pages, out_len
        c_void_p, c_void_p, c_int, c_void_p,  # k_out, v_out, dtype, stream
    ]),
    "ivakv_decode_workspace_size": (c_int, [
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, POINTER(c_size_t),
    ]),
    "ivakv_decode_attn": (c_int, _DECODE_ARGS),
    "ivakv_decode_attn_partial": (c_int, _DECODE_ARGS),
    "ivakv_decode_attn_merge": (c_int, _DECODE_ARGS),
    "ivakv_decode_append_attn": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_new, v_new
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, block_tables, context_lens
        c_void_p, c_void_p, c_size_t,          # out, workspace, workspace_bytes
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_float,          # block_size, max_blocks, num_pages, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_append_fp8": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,  # k_new, v_new, strides
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, k_scale, v_scale
        c_void_p, c_int, c_int, c_int, c_int, c_int,  # slots, n_tok, Hkv, D, bs, num_pages
        c_int, c_void_p,                         # dtype, stream
    ]),
    "ivakv_gather_fp8": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, k_scale, v_scale
        c_void_p, c_void_p,                      # block_tables, context_lens
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,  # B, max_blocks, Hkv, D, bs, pages, out_len
        c_void_p, c_void_p, c_int, c_void_p,     # k_out, v_out, dtype, stream
    ]),
    "ivakv_decode_attn_fp8": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
        c_void_p, c_void_p,                    # k_scale, v_scale
        c_void_p, c_void_p,                    # block_tables, context_lens
        c_void_p, c_void_p, c_size_t,          # out, workspace, workspace_bytes
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_float,          # block_size, max_blocks, num_pages, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_decode_append_attn_fp8": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_new, v_new
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, k_scale, v_scale
        c_void_p, c_void_p,                    # block_tables, context_lens
        c_void_p, c_void_p, c_size_t,          # out, workspace, workspace_bytes
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_float,          # block_size, max_blocks, num_pages, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_rope": (c_int, [
        c_void_p, c_int64, c_int64, c_void_p,  # x, token / head strides, positions
        c_int, c_int, c_int, c_float, c_int, c_void_p,  # n_tok, H, D, theta, dtype, stream
    ]),
    "ivakv_append_rope": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,  # k_new, v_new, strides
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, slot_mapping, positions
        c_int, c_int, c_int, c_int, c_int,     # n_tok, Hkv, D, block_size, num_pages
        c_float, c_int, c_void_p,              # theta, dtype, stream
    ]),
    "ivakv_append_rope_fp8": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,  # k_new, v_new, strides
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, k_scale, v_scale
        c_void_p, c_void_p,                    # slot_mapping, positions
        c_int, c_int, c_int, c_int, c_int,     # n_tok, Hkv, D, block_size, num_pages
        c_float, c_int, c_void_p,              # theta, dtype, stream
    ]),
    "ivakv_copy_pages": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p,  # k_pool, v_pool, k_scale, v_scale
        c_void_p, c_void_p, c_int, c_int,      # src_pages, dst_pages, n_moves, num_pages
        c_int, c_int, c_int, c_int, c_void_p,  # Hkv, D, block_size, elem_bytes, stream
    ]),
    "ivakv_decode_append_attn_noalloc": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_new, v_new
        c_void_p, c_void_p,                    # k_pool, v_pool
        c_void_p, c_void_p, c_void_p,          # block_tables, context_lens, out
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_float,          # block_size, max_blocks, num_pages, scale
        c_int, c_int, c_int, c_void_p,         # window, n_sink, dtype, stream
    ]),
    "ivakv_prefill_attn_fp8": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
        c_void_p, c_void_p,                    # k_scale, v_scale
        c_void_p, c_void_p, c_void_p,          # block_tables, context_lens, query_start
        c_int, c_void_p,                       # n_tok, out
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_int, c_float,   # block_size, max_blocks, num_pages, max_query_len, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_prefill_attn": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
        c_void_p, c_void_p, c_void_p,          # block_tables, context_lens, query_start
        c_int, c_void_p,                       # n_tok, out
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_int, c_float,   # block_size, max_blocks, num_pages, max_query_len, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_prefill_split_workspace_size": (c_int, [
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, POINTER(c_size_t),       # max_query_len, dtype, bytes
    ]),
    "ivakv_prefill_attn_split": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
        c_void_p, c_void_p, c_void_p,          # block_tables, context_lens, query_start
        c_int, c_void_p,                       # n_tok, out
        c_void_p, c_size_t,                    # workspace, workspace_bytes
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_int, c_float,   # block_size, max_blocks, num_pages, max_query_len, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_prefill_attn_split_fp8": (c_int, [
        c_void_p, c_void_p, c_void_p,          # q, k_pool, v_pool
        c_void_p, c_void_p,                    # k_scale, v_scale
        c_void_p, c_void_p, c_void_p,          # block_tables, context_lens, query_start
        c_int, c_void_p,                       # n_tok, out
        c_void_p, c_size_t,                    # workspace, workspace_bytes
        c_int, c_int, c_int, c_int,            # batch, num_q_heads, num_kv_heads, head_dim
        c_int, c_int, c_int, c_int, c_float,   # block_size, max_blocks, num_pages, max_query_len, scale
        c_int, c_int, c_int,                   # window, n_sink, dtype
        c_void_p,                              # stream
    ]),
    "ivakv_index_gather": (c_int, [
        c_void_p, c_int64, c_int64, c_int64, c_int64,  # kv + strides
        c_void_p, c_int,                             # indices, n_idx
        c_int, c_int, c_int, c_int,                  # B, H, S, D
        c_void_p, c_int, c_void_p,                   # out, dtype, stream
    ]),
    "ivakv_index_scatter": (c_int, [
        c_void_p, c_int64, c_int64, c_int64, c_int64,  # kv + strides
        c_void_p, c_int,                             # indices, n_idx
        c_void_p, c_int64, c_int64, c_int64, c_int64,  # values + strides
        c_int, c_int, c_int, c_int,                  # B, H, S, D
        c_int, c_void_p,                             # dtype, stream
    ]),
}


class IvakvError(RuntimeError):
    """A libivakv entry point returned a non-zero status."""

    def __init__(self, func: str, status: int, message: str):
        super().__init__(f"{func} failed with status {status}: {message}")
        self.func = func
        self.status = status
        self.message = message


_LIB: Optional[ctypes.CDLL] = None


def library_path() -> Path:
    env = os.environ.get("IVAKV_LIB")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "libivakv.so"


def lib() -> ctypes.CDLL:
    """Loads (once) and returns the bound library; raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"libivakv.so not found at {path}: build it first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.ivakv_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    _LIB = handle
    return handle


def last_error() -> str:
    msg = lib().ivakv_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Calls entry point ``name``; raises IvakvError on a non-zero status."""
    status = getattr(lib(), name)(*args)
    if status != OK:
        raise IvakvError(name, status, last_error())
