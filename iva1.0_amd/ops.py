"""Tensor-level paged KV ops on the HIP library (the operator API of this package).

Every function here validates shapes on the host, then enqueues libivakv
kernels on the current HIP stream of the tensors' device.  Nothing falls back
to another implementation: a CPU tensor, an unsupported dtype or a missing
library raises.

Pool layout (X = 16 bytes / element size, e.g. 8 for fp16, 4 for fp32, 16 for fp8):
    k_pool: [num_pages, Hkv, D // X, block_size, X]
    v_pool: [num_pages, Hkv, D, block_size]
FP8 pools (torch.float8_e4m3fn) carry one fp32 scaling factor per (slot, kv head):
    k_scale, v_scale: [num_pages, Hkv, block_size]; a row reads back as code / scale.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import torch

from . import _abi

_DTYPE_CODES = {torch.float32: _abi.F32, torch.float16: _abi.F16, torch.bfloat16: _abi.BF16}


FP8 = torch.float8_e4m3fn


def is_fp8(t: torch.Tensor) -> bool:
    return t.dtype == FP8


def scale_shape(num_pages: int, num_kv_heads: int, block_size: int = 16) -> Tuple[int, int, int]:
    """Shape of the per-(slot, kv head) scaling factors of an FP8 pool."""
    return (num_pages, num_kv_heads, block_size)


def _scales(k_pool, k_scale, v_scale):
    """Checks the scaling-factor tensors of an FP8 pool pair."""
    if k_scale is None or v_scale is None:
        raise ValueError("FP8 pools need k_scale and v_scale ([num_pages, Hkv, block_size] fp32)")
    shape = (k_pool.shape[0], k_pool.shape[1], k_pool.shape[3])
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if tuple(t.shape) != shape or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor of shape {shape}")
        if t.device != k_pool.device:
            raise RuntimeError(f"{name} on {t.device}, pools on {k_pool.device}")
    return k_scale, v_scale


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported KV dtype {dtype}; expected float32, float16 or bfloat16") from None


def chunk_elems(dtype: torch.dtype) -> int:
    """Elements per 16-byte chunk (the innermost K-page dimension)."""
    return 16 // torch.empty((), dtype=dtype).element_size()


def pool_shapes(num_pages: int, num_kv_heads: int, head_dim: int, block_size: int,
                dtype: torch.dtype) -> Tuple[Tuple[int, ...], Tuple[int, ...]]:
    """Shapes of (k_pool, v_pool) for one layer.  For FP8 pools the V tile's 16 * D
    bytes are not in (dim, key) order but in the walk's order [d%16][key/4][d/16][key%4]
    (ivakv_internal.h fp8_v_offset); only the kernels read or write them."""
    x = chunk_elems(dtype)
    if head_dim % x:
        raise ValueError(f"head_dim {head_dim} must be a multiple of {x} for {dtype}")
    return ((num_pages, num_kv_heads, head_dim // x, block_size, x),
            (num_pages, num_kv_heads, head_dim, block_size))


def pool_geometry(k_pool: torch.Tensor, v_pool: torch.Tensor) -> Tuple[int, int, int, int]:
    """(num_pages, Hkv, head_dim, block_size) of a pool pair; checks the layout."""
    if k_pool.dim() != 5 or v_pool.dim() != 4:
        raise ValueError("k_pool must be [P, Hkv, D/X, bs, X] and v_pool [P, Hkv, D, bs]")
    num_pages, hkv, nch, bs, x = k_pool.shape
    if x != chunk_elems(k_pool.dtype):
        raise ValueError(f"k_pool innermost dim {x} != 16-byte chunk {chunk_elems(k_pool.dtype)}")
    head_dim = nch * x
    if tuple(v_pool.shape) != (num_pages, hkv, head_dim, bs):
        raise ValueError(f"v_pool shape {tuple(v_pool.shape)} != {(num_pages, hkv, head_dim, bs)}")
    if k_pool.dtype != v_pool.dtype:
        raise TypeError("k_pool and v_pool dtypes differ")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    return num_pages, hkv, head_dim, bs


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(f"paged KV ops run on the GPU only; got a tensor on {t.device}")
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _capturing(dev: torch.device) -> bool:
    """True while the device's current stream is being captured into a HIP graph, when
    no host read of device data is allowed (the kernels' own bounds checks then stand)."""
    with torch.cuda.device(dev):
        return torch.cuda.is_current_stream_capturing()


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    return t.contiguous()


def _buffer(t: torch.Tensor, dev: torch.device, name: str) -> torch.Tensor:
    """A caller-supplied output or workspace: on the op's device and contiguous (the
    library writes its data pointer's whole extent)."""
    if t.device != dev:
        raise RuntimeError(f"{name} is on {t.device}; the op runs on {dev}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
              slot_mapping: torch.Tensor, k_scale: Optional[torch.Tensor] = None,
              v_scale: Optional[torch.Tensor] = None,
              rope_positions: Optional[torch.Tensor] = None, rope_theta: float = 10000.0) -> None:
    """Scatters rows ``k_new[t], v_new[t]`` ([n_tok, Hkv, D], last dim contiguous) into
    ``slot_mapping[t]`` of the pools, in place.  A slot of -1 (or any slot outside the
    pool) leaves the pools untouched for that token.  FP8 pools quantize each (token,
    kv head) row with its own scaling factor, written to ``k_scale`` / ``v_scale``.
    With ``rope_positions`` (int32 ``[n_tok]``) every K row is rotated at its position on
    the way in (:func:`rope_`), fused into the append kernel.

    Paged counterpart of ``KVCache.update`` (src/core/rope_kv.py:98-110) and the
    ``torch.cat`` append of ``AttentionTorch.forward`` (src/core/attention.py:61-63).
    """
    if is_fp8(k_pool):
        return _append_fp8(k_new, v_new, k_pool, v_pool, slot_mapping, k_scale, v_scale,
                           rope_positions, rope_theta)
    dev = _require_gpu(k_new, v_new, k_pool, v_pool, slot_mapping)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    if k_new.dim() != 3 or tuple(k_new.shape) != tuple(v_new.shape):
        raise ValueError(f"k_new/v_new must be [n_tok, Hkv, D]; got {tuple(k_new.shape)} and {tuple(v_new.shape)}")
    n_tok = k_new.shape[0]
    if k_new.shape[1:] != (hkv, head_dim):
        raise ValueError(f"new rows are {tuple(k_new.shape[1:])}, pool holds ({hkv}, {head_dim})")
    if k_new.dtype != k_pool.dtype or v_new.dtype != k_pool.dtype:
        raise TypeError(f"new rows dtype {k_new.dtype}/{v_new.dtype} != pool dtype {k_pool.dtype}")
    slot_mapping = _i32(slot_mapping, "slot_mapping").reshape(-1)
    if slot_mapping.numel() != n_tok:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {n_tok} tokens")
    if n_tok == 0:
        return
    if k_new.stride(2) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(2) != 1:
        v_new = v_new.contiguous()
    if rope_positions is not None:
        pos = _i32(rope_positions, "rope_positions").reshape(-1)
        if pos.numel() != n_tok or pos.device != dev:
            raise ValueError(f"rope_positions must be {n_tok} int32 values on {dev}")
        _abi.call("ivakv_append_rope", k_new.data_ptr(), v_new.data_ptr(),
                  k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1),
                  k_pool.data_ptr(), v_pool.data_ptr(), slot_mapping.data_ptr(), pos.data_ptr(),
                  n_tok, hkv, head_dim, bs, num_pages, float(rope_theta),
                  dtype_code(k_pool.dtype), _stream(dev))
        return
    _abi.call("ivakv_append", k_new.data_ptr(), v_new.data_ptr(),
              k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1),
              k_pool.data_ptr(), v_pool.data_ptr(), slot_mapping.data_ptr(),
              n_tok, hkv, head_dim, bs, num_pages, dtype_code(k_pool.dtype), _stream(dev))


def kv_gather(k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
              context_lens: torch.Tensor, out_len: Optional[int] = None,
              out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
              k_scale: Optional[torch.Tensor] = None, v_scale: Optional[torch.Tensor] = None,
              out_dtype: Optional[torch.dtype] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gathers each sequence's pages back into contiguous ``[B, Hkv, out_len, D]`` K and V
    (pool dtype).  Rows at or beyond ``context_lens[b]`` are zero.  ``out_len`` defaults to
    ``block_tables.shape[1] * block_size``.  FP8 pools are dequantized (code / scale) into
    ``out_dtype`` (default float16).

    Paged counterpart of ``KVCache.get_slice`` (src/core/rope_kv.py:136-137) and the gather
    branch of ``KVOpsTriton`` (src/kernels_t/kv_ops_triton.py:111-123).
    """
    if is_fp8(k_pool):
        return _gather_fp8(k_pool, v_pool, block_tables, context_lens, out_len, out, k_scale,
                           v_scale, out_dtype or torch.float16)
    dev = _require_gpu(k_pool, v_pool, block_tables, context_lens)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    block_tables = _i32(block_tables, "block_tables")
    context_lens = _i32(context_lens, "context_lens").reshape(-1)
    if block_tables.dim() != 2 or block_tables.shape[0] != context_lens.numel():
        raise ValueError("block_tables must be [B, max_blocks] with B == len(context_lens)")
    batch, max_blocks = block_tables.shape
    if out_len is None:
        out_len = max_blocks * bs
    shape = (batch, hkv, out_len, head_dim)
    if out is None:
        k_out = torch.empty(shape, dtype=k_pool.dtype, device=dev)
        v_out = torch.empty(shape, dtype=k_pool.dtype, device=dev)
    else:
        k_out, v_out = out
        for t in (k_out, v_out):
            if tuple(t.shape) != shape or t.dtype != k_pool.dtype or not t.is_contiguous():
                raise ValueError(f"gather outputs must be contiguous {shape} {k_pool.dtype}")
            _buffer(t, dev, "gather output")
    _abi.call("ivakv_gather", k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
              context_lens.data_ptr(), batch, max_blocks, hkv, head_dim, bs, num_pages, out_len,
              k_out.data_ptr(), v_out.data_ptr(), dtype_code(k_pool.dtype), _stream(dev))
    return k_out, v_out


_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}


def decode_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                           block_size: int, max_blocks: int, window: int = 0, n_sink: int = 0,
                           partition_pages: int = 0) -> int:
    """Workspace bytes :func:`paged_decode_attention` needs (0 when no sequence spans more
    than one partition).  The workspace needs no initialisation."""
    import ctypes
    out = ctypes.c_size_t(0)
    _abi.call("ivakv_decode_workspace_size", batch, num_q_heads, num_kv_heads, head_dim,
              block_size, max_blocks, window, n_sink, partition_pages, ctypes.byref(out))
    return int(out.value)


# Split prefill (ivakv_prefill_attn_split) by default, up to the split path's largest
# batch, when a walk may exceed SPLIT_MIN_KEYS keys (a chunk late in a long context:
# 2-3.4x on one 512-token chunk at 8k-64k) or when the launch's work bound, query rows x
# query heads x keys, reaches SPLIT_MIN_WORK (enough work that the persistent grid's
# longest-first order pays for the plan launch: the ragged prefill chunks of a
# continuous-batching step take 25 % less time split, and 16 x 512 rows at 2048 keys take
# the same time either way; shorter prefills are 2-11 us slower split), or when a walk
# may pass SPLIT_FEW_BLOCKS_KEYS keys and the single launch would have fewer than
# SPLIT_FEW_BLOCKS workgroups of 256 query rows (x query heads of a kv head), half the
# CUs: then most CUs would idle while a few walk the whole context (one sequence, a
# 128-row chunk at 4096 keys: 148 against 62 us split; a 16-row chunk at 2048 keys: 58
# against 40 us; four 128-row chunks at 2048 keys, 64 workgroups: 81 against 61 us).
# With 128-256 such workgroups the single launch stays ahead (four 512-row chunks at
# 2048 keys: 99 against 125 us), and so it does at 1024 keys (33 against 38 us).
SPLIT_MIN_KEYS = 4096
SPLIT_MIN_WORK = 1 << 28
SPLIT_FEW_BLOCKS_KEYS = 2048
SPLIT_FEW_BLOCKS = 128
SPLIT_MAX_BATCH = 2048
SPLIT_MAX_KV_HEADS = 32767


def prefill_split_default(batch: int, num_q_heads: int, num_kv_heads: int, n_tok: int,
                          max_query_len: int, max_blocks: int, block_size: int,
                          window: int = 0, n_sink: int = 0) -> bool:
    """:func:`paged_prefill_attention`'s default for ``split``: within the split path's
    batch and kv-head limits, when the longest walk the table allows (its width in keys,
    or window + chunk + sinks) exceeds SPLIT_MIN_KEYS, when query rows x query heads x
    those keys reaches SPLIT_MIN_WORK, or when that walk reaches SPLIT_FEW_BLOCKS_KEYS
    and the single launch would have fewer than SPLIT_FEW_BLOCKS row-block workgroups
    (256 rows of a kv head's query heads each, counted for chunks of max_query_len)."""
    keys = max_blocks * block_size
    if window and window > 0:
        keys = min(keys, window + max_query_len + max(n_sink, 0))
    group = max(num_q_heads // max(num_kv_heads, 1), 1)
    row_blocks = batch * num_kv_heads * (-(-max_query_len * group // 256))
    return batch <= SPLIT_MAX_BATCH and num_kv_heads <= SPLIT_MAX_KV_HEADS and (
        keys > SPLIT_MIN_KEYS or n_tok * num_q_heads * keys >= SPLIT_MIN_WORK
        or (keys >= SPLIT_FEW_BLOCKS_KEYS and row_blocks < SPLIT_FEW_BLOCKS))


def prefill_split_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int,
                                  head_dim: int, max_query_len: int,
                                  dtype: torch.dtype) -> int:
    """Workspace bytes of :func:`paged_prefill_attention` with ``split=True`` (its plan
    and 512 fp32 row-block partials).  The workspace needs no initialisation."""
    import ctypes
    out = ctypes.c_size_t(0)
    _abi.call("ivakv_prefill_split_workspace_size", batch, num_q_heads, num_kv_heads, head_dim,
              max_query_len, dtype_code(dtype), ctypes.byref(out))
    return int(out.value)


# Workspaces replaced by larger ones stay allocated: a HIP graph captured with one keeps
# its address, and freeing it would let the caching allocator hand that memory out
# while the graph still writes there.
_RETIRED_WORKSPACES: List[torch.Tensor] = []


def _workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The op-owned workspace of (device, current stream), grown to at least nbytes.
    A replacement is at least twice the size it replaces, so the retired workspaces
    together stay smaller than the live one."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        grown = 1
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
            grown = 2 * ws.numel()
        ws = torch.empty(max(nbytes, grown), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


def _decode(entry: str, q, k_pool, v_pool, block_tables, context_lens, scale, window, n_sink,
            partition_pages, out, workspace, scales=None):
    dev = _require_gpu(q, k_pool, v_pool, block_tables, context_lens)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    if q.dim() != 3 or q.shape[2] != head_dim:
        raise ValueError(f"q must be [B, Hq, {head_dim}]; got {tuple(q.shape)}")
    if scales is not None:
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"FP8 pools take float16 or bfloat16 queries, got {q.dtype}")
    elif q.dtype != k_pool.dtype:
        raise TypeError(f"q dtype {q.dtype} != pool dtype {k_pool.dtype}")
    elif is_fp8(k_pool):
        raise ValueError("FP8 pools need k_scale / v_scale")
    batch, hq, _ = q.shape
    block_tables = _i32(block_tables, "block_tables")
    context_lens = _i32(context_lens, "context_lens").reshape(-1)
    if block_tables.dim() != 2 or block_tables.shape[0] != batch or context_lens.numel() != batch:
        raise ValueError("block_tables must be [B, max_blocks] and context_lens [B]")
    max_blocks = block_tables.shape[1]
    q = q.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    window = int(window) if window else 0
    n_sink = int(n_sink) if n_sink else 0
    partition_pages = int(partition_pages) if partition_pages else 0
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped and typed like q")
    _buffer(out, dev, "out")
    nbytes = decode_workspace_bytes(batch, hq, hkv, head_dim, bs, max_blocks, window, n_sink,
                                    partition_pages)
    if workspace is None:
        workspace = _workspace(dev, nbytes)
    elif workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace has {workspace.numel() * workspace.element_size()} bytes, "
                         f"{nbytes} needed")
    _buffer(workspace, dev, "workspace")
    if scales is not None:
        _abi.call(entry, q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                  scales[0].data_ptr(), scales[1].data_ptr(), block_tables.data_ptr(),
                  context_lens.data_ptr(), out.data_ptr(), workspace.data_ptr(),
                  workspace.numel() * workspace.element_size(), batch, hq, hkv, head_dim, bs,
                  max_blocks, num_pages, float(scale), window, n_sink, dtype_code(q.dtype),
                  _stream(dev))
        return out
    _abi.call(entry, q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
              context_lens.data_ptr(), out.data_ptr(), workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), batch, hq, hkv, head_dim, bs,
              max_blocks, num_pages, float(scale), window, n_sink, partition_pages,
              dtype_code(q.dtype), _stream(dev))
    return out


def paged_decode_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor,
                           scale: Optional[float] = None, window: Optional[int] = None,
                           n_sink: int = 0, partition_pages: Optional[int] = None,
                           out: Optional[torch.Tensor] = None,
                           workspace: Optional[torch.Tensor] = None,
                           k_scale: Optional[torch.Tensor] = None,
                           v_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Single-query attention over paged K/V: ``q`` is ``[B, Hq, D]``; returns ``[B, Hq, D]``.

    Sequence b attends to positions ``j < context_lens[b]`` that lie in the sliding window
    ``j >= L - window`` (all when ``window`` is None/0) or among the first ``n_sink``
    attention-sink positions.  Query head h reads KV head ``h // (Hq // Hkv)``.
    ``scale`` defaults to ``1/sqrt(D)`` as in ``AttentionTorch`` (src/core/attention.py:35).

    FP8 pools (``torch.float8_e4m3fn`` with ``k_scale`` / ``v_scale``) take fp16 or bf16
    queries and attend over the dequantized keys and values.

    Replaces the cache branch of ``AttentionTorch.forward`` (src/core/attention.py:77-102).
    """
    if is_fp8(k_pool):
        if partition_pages:
            raise ValueError("FP8 pools use the stream walk (partition_pages must be 0/None)")
        return _decode("ivakv_decode_attn_fp8", q, k_pool, v_pool, block_tables, context_lens,
                       scale, window, n_sink, None, out, workspace,
                       scales=_scales(k_pool, k_scale, v_scale))
    return _decode("ivakv_decode_attn", q, k_pool, v_pool, block_tables, context_lens, scale,
                   window, n_sink, partition_pages, out, workspace)


def paged_decode_attention_partial(q, k_pool, v_pool, block_tables, context_lens, scale=None,
                                   window=None, n_sink=0, partition_pages=None, out=None,
                                   workspace=None) -> torch.Tensor:
    """First half of :func:`paged_decode_attention` (the paged walk); see include/ivakv.h."""
    return _decode("ivakv_decode_attn_partial", q, k_pool, v_pool, block_tables, context_lens,
                   scale, window, n_sink, partition_pages, out, workspace)


def paged_decode_attention_merge(q, k_pool, v_pool, block_tables, context_lens, scale=None,
                                 window=None, n_sink=0, partition_pages=None, out=None,
                                 workspace=None) -> torch.Tensor:
    """Second half of :func:`paged_decode_attention` (log-sum-exp merge of partitions)."""
    return _decode("ivakv_decode_attn_merge", q, k_pool, v_pool, block_tables, context_lens,
                   scale, window, n_sink, partition_pages, out, workspace)


def paged_decode_append_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                                  k_pool: torch.Tensor, v_pool: torch.Tensor,
                                  block_tables: torch.Tensor, context_lens: torch.Tensor,
                                  scale: Optional[float] = None, window: Optional[int] = None,
                                  n_sink: int = 0, out: Optional[torch.Tensor] = None,
                                  workspace: Optional[torch.Tensor] = None,
                                  k_scale: Optional[torch.Tensor] = None,
                                  v_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One decode step in one op: the new token of sequence b sits at position
    ``context_lens[b] - 1``; its rows ``k_new[b], v_new[b]`` ([B, Hkv, D]) are written to
    that position's slot and attended together with the earlier positions in the pages.
    Same result as :func:`kv_append` of those rows followed by
    :func:`paged_decode_attention`, in two launches (no separate append kernel).

    FP8 pools (``torch.float8_e4m3fn`` with ``k_scale`` / ``v_scale``): ``q``, ``k_new``
    and ``v_new`` are fp16 or bf16; the new rows are quantized as :func:`kv_append` does
    (same codes and factors) and attended as their dequantized values.

    Fuses the append and the scoring of ``AttentionTorch.forward`` with a cache
    (src/core/attention.py:61-102).
    """
    dev = _require_gpu(q, k_new, v_new, k_pool, v_pool, block_tables, context_lens)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    if q.dim() != 3 or q.shape[2] != head_dim:
        raise ValueError(f"q must be [B, Hq, {head_dim}]; got {tuple(q.shape)}")
    batch, hq, _ = q.shape
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if tuple(t.shape) != (batch, hkv, head_dim):
            raise ValueError(f"{name} must be [{batch}, {hkv}, {head_dim}]; got {tuple(t.shape)}")
    fp8 = is_fp8(k_pool)
    for t in (q, k_new, v_new):
        if fp8 and t.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"FP8 pools take float16 or bfloat16 q / k_new / v_new; got {t.dtype}")
        if t.dtype != (q.dtype if fp8 else k_pool.dtype):
            raise TypeError(f"dtype {t.dtype} != {q.dtype if fp8 else k_pool.dtype}")
    scales = _scales(k_pool, k_scale, v_scale) if fp8 else None
    block_tables = _i32(block_tables, "block_tables")
    context_lens = _i32(context_lens, "context_lens").reshape(-1)
    if block_tables.dim() != 2 or block_tables.shape[0] != batch or context_lens.numel() != batch:
        raise ValueError("block_tables must be [B, max_blocks] and context_lens [B]")
    max_blocks = block_tables.shape[1]
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    window = int(window) if window else 0
    n_sink = int(n_sink) if n_sink else 0
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped and typed like q")
    _buffer(out, dev, "out")
    nbytes = decode_workspace_bytes(batch, hq, hkv, head_dim, bs, max_blocks, window, n_sink)
    if workspace is None:
        workspace = _workspace(dev, nbytes)
    elif workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace has {workspace.numel() * workspace.element_size()} bytes, "
                         f"{nbytes} needed")
    _buffer(workspace, dev, "workspace")
    if fp8:
        _abi.call("ivakv_decode_append_attn_fp8", q.data_ptr(), k_new.data_ptr(),
                  v_new.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), scales[0].data_ptr(),
                  scales[1].data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                  out.data_ptr(), workspace.data_ptr(),
                  workspace.numel() * workspace.element_size(), batch, hq, hkv, head_dim, bs,
                  max_blocks, num_pages, float(scale), window, n_sink, dtype_code(q.dtype),
                  _stream(dev))
        return out
    _abi.call("ivakv_decode_append_attn", q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
              k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
              context_lens.data_ptr(), out.data_ptr(), workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), batch, hq, hkv, head_dim, bs,
              max_blocks, num_pages, float(scale), window, n_sink, dtype_code(q.dtype),
              _stream(dev))
    return out


def _append_fp8(k_new, v_new, k_pool, v_pool, slot_mapping, k_scale, v_scale,
                rope_positions=None, rope_theta=10000.0) -> None:
    dev = _require_gpu(k_new, v_new, k_pool, v_pool, slot_mapping)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    k_scale, v_scale = _scales(k_pool, k_scale, v_scale)
    if k_new.dim() != 3 or tuple(k_new.shape) != tuple(v_new.shape):
        raise ValueError(f"k_new/v_new must be [n_tok, Hkv, D]; got {tuple(k_new.shape)} and {tuple(v_new.shape)}")
    n_tok = k_new.shape[0]
    if k_new.shape[1:] != (hkv, head_dim):
        raise ValueError(f"new rows are {tuple(k_new.shape[1:])}, pool holds ({hkv}, {head_dim})")
    if k_new.dtype != v_new.dtype:
        raise TypeError("k_new and v_new dtypes differ")
    code = dtype_code(k_new.dtype)
    slot_mapping = _i32(slot_mapping, "slot_mapping").reshape(-1)
    if slot_mapping.numel() != n_tok:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {n_tok} tokens")
    if n_tok == 0:
        return
    if k_new.stride(2) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(2) != 1:
        v_new = v_new.contiguous()
    if rope_positions is not None:
        pos = _i32(rope_positions, "rope_positions").reshape(-1)
        if pos.numel() != n_tok or pos.device != dev:
            raise ValueError(f"rope_positions must be {n_tok} int32 values on {dev}")
        _abi.call("ivakv_append_rope_fp8", k_new.data_ptr(), v_new.data_ptr(),
                  k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1),
                  k_pool.data_ptr(), v_pool.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
                  slot_mapping.data_ptr(), pos.data_ptr(), n_tok, hkv, head_dim, bs, num_pages,
                  float(rope_theta), code, _stream(dev))
        return
    _abi.call("ivakv_append_fp8", k_new.data_ptr(), v_new.data_ptr(),
              k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1),
              k_pool.data_ptr(), v_pool.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
              slot_mapping.data_ptr(), n_tok, hkv, head_dim, bs, num_pages, code, _stream(dev))


def _gather_fp8(k_pool, v_pool, block_tables, context_lens, out_len, out, k_scale, v_scale,
                out_dtype):
    dev = _require_gpu(k_pool, v_pool, block_tables, context_lens)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    k_scale, v_scale = _scales(k_pool, k_scale, v_scale)
    block_tables = _i32(block_tables, "block_tables")
    context_lens = _i32(context_lens, "context_lens").reshape(-1)
    if block_tables.dim() != 2 or block_tables.shape[0] != context_lens.numel():
        raise ValueError("block_tables must be [B, max_blocks] with B == len(context_lens)")
    batch, max_blocks = block_tables.shape
    if out_len is None:
        out_len = max_blocks * bs
    shape = (batch, hkv, out_len, head_dim)
    if out is None:
        k_out = torch.empty(shape, dtype=out_dtype, device=dev)
        v_out = torch.empty(shape, dtype=out_dtype, device=dev)
    else:
        k_out, v_out = out
        for t in (k_out, v_out):
            if tuple(t.shape) != shape or not t.is_contiguous() or t.dtype != k_out.dtype:
                raise ValueError(f"gather outputs must be contiguous {shape}, one dtype")
            _buffer(t, dev, "gather output")
    _abi.call("ivakv_gather_fp8", k_pool.data_ptr(), v_pool.data_ptr(), k_scale.data_ptr(),
              v_scale.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(), batch,
              max_blocks, hkv, head_dim, bs, num_pages, out_len, k_out.data_ptr(),
              v_out.data_ptr(), dtype_code(k_out.dtype), _stream(dev))
    return k_out, v_out


def paged_prefill_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                            block_tables: torch.Tensor, context_lens: torch.Tensor,
                            query_start: torch.Tensor, scale: Optional[float] = None,
                            window: Optional[int] = None, n_sink: int = 0,
                            max_query_len: Optional[int] = None,
                            out: Optional[torch.Tensor] = None,
                            k_scale: Optional[torch.Tensor] = None,
                            v_scale: Optional[torch.Tensor] = None,
                            split: Optional[bool] = None,
                            workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal multi-query attention of chunks of new tokens over paged K/V.

    ``q`` is ``[n_tok, Hq, D]``; the rows of sequence b are
    ``query_start[b] .. query_start[b+1]-1`` (int32 ``[B+1]``) and sit at absolute
    positions ``L - n_b .. L - 1`` with ``L = context_lens[b]``.  Their K/V must already
    be in the pages (:func:`kv_append`).  Row at position p attends to keys ``j <= p``
    within the window (``j > p - window``) or among the first ``n_sink`` positions.
    Returns ``[n_tok, Hq, D]``.  ``max_query_len`` (>= every chunk length) sizes the
    launch; when omitted it is read back from ``query_start`` (a device sync), and
    ``query_start`` is then checked: 0-based, non-decreasing, ending at ``n_tok``.  The
    kernel skips a sequence whose rows do not lie inside ``q`` either way.
    FP8 pools (``torch.float8_e4m3fn`` with ``k_scale`` / ``v_scale``) take fp16 or bf16
    queries; keys and values are dequantized (code / sf, rounded to the query dtype)
    on their way into LDS.
    ``split`` cuts every row block's walk along the keys into segments sized to the
    batch's work per CU (``ivakv_prefill_attn_split``: plan, persistent grid, merge),
    so a chunk late in a long context no longer runs as a few long serial walks.  The
    default (None) splits when a walk may exceed 4096 keys (from the block table's width,
    or the window) or when rows x query heads x keys reaches 2^28; ``workspace``
    (:func:`prefill_split_workspace_bytes`) is then allocated and kept per device and
    stream when omitted.

    Replaces ``AttentionTorch.forward`` with a cache and ``seq_len > 1``
    (src/core/attention.py:61-102), with the causal, window and sink masks
    (attention.py:79-93,115-148) taken at absolute positions.
    """
    dev = _require_gpu(q, k_pool, v_pool, block_tables, context_lens, query_start)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    if q.dim() != 3 or q.shape[2] != head_dim:
        raise ValueError(f"q must be [n_tok, Hq, {head_dim}]; got {tuple(q.shape)}")
    fp8 = is_fp8(k_pool)
    if fp8:
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"FP8 pools take float16 or bfloat16 queries, got {q.dtype}")
        scales = _scales(k_pool, k_scale, v_scale)
    elif q.dtype != k_pool.dtype:
        raise TypeError(f"q dtype {q.dtype} != pool dtype {k_pool.dtype}")
    hq = q.shape[1]
    block_tables = _i32(block_tables, "block_tables")
    context_lens = _i32(context_lens, "context_lens").reshape(-1)
    query_start = _i32(query_start, "query_start").reshape(-1)
    batch = context_lens.numel()
    if block_tables.dim() != 2 or block_tables.shape[0] != batch:
        raise ValueError("block_tables must be [B, max_blocks] with B == len(context_lens)")
    if query_start.numel() != batch + 1:
        raise ValueError(f"query_start must have B+1 = {batch + 1} entries")
    if max_query_len is None:
        if _capturing(dev):
            raise ValueError("max_query_len is required under HIP-graph capture (the host "
                             "cannot read query_start then)")
        qs = query_start.tolist()
        if qs[0] != 0 or qs[-1] != q.shape[0] or any(b < a for a, b in zip(qs, qs[1:])):
            raise ValueError(f"query_start must rise from 0 to n_tok = {q.shape[0]}; got "
                             f"{qs if len(qs) <= 8 else qs[:4] + ['...'] + qs[-4:]}")
        max_query_len = max((b - a for a, b in zip(qs, qs[1:])), default=0)
    q = q.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    window = int(window) if window else 0
    n_sink = int(n_sink) if n_sink else 0
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped and typed like q")
    _buffer(out, dev, "out")
    max_blocks = block_tables.shape[1]
    if split is None:
        split = prefill_split_default(batch, hq, hkv, q.shape[0], int(max_query_len), max_blocks,
                                      bs, window, n_sink)
    if split:
        nbytes = prefill_split_workspace_bytes(batch, hq, hkv, head_dim, int(max_query_len),
                                               q.dtype)
        if workspace is None:
            workspace = _workspace(dev, nbytes)
        elif workspace.numel() * workspace.element_size() < nbytes:
            raise ValueError(f"workspace has {workspace.numel() * workspace.element_size()} "
                             f"bytes, {nbytes} needed")
        _buffer(workspace, dev, "workspace")
        ws = (workspace.data_ptr(), workspace.numel() * workspace.element_size())
        if fp8:
            _abi.call("ivakv_prefill_attn_split_fp8", q.data_ptr(), k_pool.data_ptr(),
                      v_pool.data_ptr(), scales[0].data_ptr(), scales[1].data_ptr(),
                      block_tables.data_ptr(), context_lens.data_ptr(), query_start.data_ptr(),
                      q.shape[0], out.data_ptr(), *ws, batch, hq, hkv, head_dim, bs, max_blocks,
                      num_pages, int(max_query_len), float(scale), window, n_sink,
                      dtype_code(q.dtype), _stream(dev))
        else:
            _abi.call("ivakv_prefill_attn_split", q.data_ptr(), k_pool.data_ptr(),
                      v_pool.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                      query_start.data_ptr(), q.shape[0], out.data_ptr(), *ws, batch, hq, hkv,
                      head_dim, bs, max_blocks, num_pages, int(max_query_len), float(scale),
                      window, n_sink, dtype_code(q.dtype), _stream(dev))
        return out
    if fp8:
        _abi.call("ivakv_prefill_attn_fp8", q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                  scales[0].data_ptr(), scales[1].data_ptr(), block_tables.data_ptr(),
                  context_lens.data_ptr(), query_start.data_ptr(), q.shape[0], out.data_ptr(),
                  batch, hq, hkv, head_dim, bs, block_tables.shape[1], num_pages,
                  int(max_query_len), float(scale), window, n_sink, dtype_code(q.dtype),
                  _stream(dev))
        return out
    _abi.call("ivakv_prefill_attn", q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
              block_tables.data_ptr(), context_lens.data_ptr(), query_start.data_ptr(),
              q.shape[0], out.data_ptr(), batch, hq, hkv, head_dim, bs, block_tables.shape[1],
              num_pages, int(max_query_len), float(scale), window, n_sink, dtype_code(q.dtype),
              _stream(dev))
    return out


def rope_(x: torch.Tensor, positions: torch.Tensor, theta: float = 10000.0) -> torch.Tensor:
    """Rotates ``x`` ([n_tok, H, D], last dim contiguous) in place at ``positions`` (int32
    ``[n_tok]``) and returns it: dims (2i, 2i+1) by the angle position * theta^(-2i/D), as
    the reference's ``RoPE.forward`` (src/core/rope_kv.py:22-50)."""
    dev = _require_gpu(x, positions)
    if x.dim() != 3 or x.shape[2] % 2 or x.stride(2) != 1:
        raise ValueError(f"x must be [n_tok, H, D] with D even and the last dim contiguous; "
                         f"got {tuple(x.shape)}")
    pos = _i32(positions, "positions").reshape(-1)
    if pos.numel() != x.shape[0]:
        raise ValueError(f"{pos.numel()} positions for {x.shape[0]} rows")
    _abi.call("ivakv_rope", x.data_ptr(), x.stride(0), x.stride(1), pos.data_ptr(), x.shape[0],
              x.shape[1], x.shape[2], float(theta), dtype_code(x.dtype), _stream(dev))
    return x


def copy_pages(k_pool: torch.Tensor, v_pool: torch.Tensor, src_pages: torch.Tensor,
               dst_pages: torch.Tensor, k_scale: Optional[torch.Tensor] = None,
               v_scale: Optional[torch.Tensor] = None) -> None:
    """Moves pages ``src_pages[i] -> dst_pages[i]`` (int32, disjoint sets) of a pool pair,
    with the FP8 scaling factors when the pools are FP8.  Every id must lie in
    ``[0, num_pages)``: checked here with one device read (``IndexError``), except under
    HIP-graph capture, where the kernel's own check skips a move outside the pool."""
    dev = _require_gpu(k_pool, v_pool, src_pages, dst_pages)
    num_pages, hkv, head_dim, bs = pool_geometry(k_pool, v_pool)
    src = _i32(src_pages, "src_pages").reshape(-1)
    dst = _i32(dst_pages, "dst_pages").reshape(-1)
    if src.numel() != dst.numel():
        raise ValueError("src_pages and dst_pages differ in length")
    if src.numel() and not _capturing(dev):
        ids = torch.cat([src, dst])
        lo, hi = (int(v) for v in torch.stack([ids.min(), ids.max()]).tolist())
        if lo < 0 or hi >= num_pages:
            raise IndexError(f"page ids in [{lo}, {hi}] outside the pool of {num_pages} pages")
    ks = vs = None
    if is_fp8(k_pool):
        ks, vs = _scales(k_pool, k_scale, v_scale)
    for start in range(0, src.numel(), 65535):
        n = min(65535, src.numel() - start)
        _abi.call("ivakv_copy_pages", k_pool.data_ptr(), v_pool.data_ptr(),
                  ks.data_ptr() if ks is not None else None,
                  vs.data_ptr() if vs is not None else None,
                  src[start:].data_ptr(), dst[start:].data_ptr(), n, num_pages, hkv, head_dim,
                  bs, k_pool.element_size(), _stream(dev))


def kv_compact(kv_cache: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """The positions of a contiguous ``[B, H, S, D]`` cache where ``mask`` is true, packed
    into ``[B, H, n_valid, D]`` (cache dtype) in position order: the compaction
    ``kv_compact_triton`` performs (src/kernels_t/kv_ops_triton.py:68-92,159-181).  The mask
    is ``[S]`` or ``[B, S]`` with identical rows (the reference sizes the output by one count
    for the whole batch, kv_ops_triton.py:165-167)."""
    if mask.dim() == 2:
        if bool((mask != mask[:1]).any()):
            raise ValueError("kv_compact needs the same mask for every sequence of the batch")
        mask = mask[0]
    if mask.dim() != 1 or mask.numel() != kv_cache.shape[2]:
        raise ValueError(f"mask must be [S] or [B, S] with S = {kv_cache.shape[2]}")
    idx = torch.nonzero(mask.to(torch.bool)).reshape(-1)
    return kv_ops(kv_cache, idx, operation="gather")


class KVOps(torch.autograd.Function):
    """``KVOpsTriton`` (src/kernels_t/kv_ops_triton.py:95-147): the index op as an autograd
    function whose backward gives no gradient to any input (an output of an input that
    requires grad is part of the graph, and backward through it stops there)."""

    @staticmethod
    def forward(ctx, kv_cache: torch.Tensor, indices: torch.Tensor,
                values: Optional[torch.Tensor] = None, operation: str = "gather") -> torch.Tensor:
        return _kv_ops(kv_cache, indices, values, operation)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        return None, None, None, None


def kv_ops(kv_cache: torch.Tensor, indices: torch.Tensor, values: Optional[torch.Tensor] = None,
           operation: str = "gather") -> torch.Tensor:
    """Index gather / scatter along the sequence axis of a contiguous ``[B, H, S, D]`` cache.

    Same signature, semantics and errors as ``kv_ops_triton``
    (src/kernels_t/kv_ops_triton.py:150-156):
      * ``"gather"``:  returns ``kv_cache[:, :, indices, :]`` as a new ``[B, H, N, D]`` tensor;
      * ``"scatter"``: returns a copy of ``kv_cache`` with ``[:, :, indices[j], :]`` replaced
        by ``values[:, :, j, :]`` (the input is not modified; with duplicate indices each
        16-byte chunk of such a row comes from one of the duplicates, unspecified which);
      * ``ValueError`` for a scatter without values or an unknown operation
        (kv_ops_triton.py:126-127,142-143).
    Differences, both deliberate: the gather output keeps the cache dtype (the reference
    allocated it in the default dtype, kv_ops_triton.py:112), and an index outside
    ``[0, S)`` raises ``IndexError`` instead of reading or writing out of bounds.
    Runs as :class:`KVOps`, as ``kv_ops_triton`` runs ``KVOpsTriton.apply``
    (kv_ops_triton.py:150-156).
    """
    return KVOps.apply(kv_cache, indices, values, operation)


def _kv_ops(kv_cache: torch.Tensor, indices: torch.Tensor, values: Optional[torch.Tensor],
            operation: str) -> torch.Tensor:
    if operation not in ("gather", "scatter"):
        raise ValueError(f"Unknown operation: {operation}")
    if operation == "scatter" and values is None:
        raise ValueError("Values tensor required for scatter operation")
    tensors = [kv_cache, indices] + ([values] if values is not None else [])
    dev = _require_gpu(*tensors)
    if kv_cache.dim() != 4:
        raise ValueError(f"kv_cache must be [B, H, S, D]; got {tuple(kv_cache.shape)}")
    batch, n_heads, seq_len, head_dim = kv_cache.shape
    idx = indices.reshape(-1).to(torch.int64).contiguous()
    n_idx = idx.numel()
    # Under HIP-graph capture the host cannot read the indices; the kernel then gathers
    # zeros for, and does not scatter, an out-of-range index.
    if n_idx and not _capturing(dev) and bool(((idx < 0) | (idx >= seq_len)).any()):
        raise IndexError(f"kv_ops index out of range for sequence length {seq_len}")
    code = dtype_code(kv_cache.dtype)
    if operation == "gather":
        out = torch.empty((batch, n_heads, n_idx, head_dim), dtype=kv_cache.dtype, device=dev)
        _abi.call("ivakv_index_gather", kv_cache.data_ptr(), *kv_cache.stride(), idx.data_ptr(),
                  n_idx, batch, n_heads, seq_len, head_dim, out.data_ptr(), code, _stream(dev))
        return out
    if tuple(values.shape) != (batch, n_heads, n_idx, head_dim):
        raise ValueError(f"values must be {(batch, n_heads, n_idx, head_dim)}; got {tuple(values.shape)}")
    if values.dtype != kv_cache.dtype:
        raise TypeError(f"values dtype {values.dtype} != cache dtype {kv_cache.dtype}")
    out = kv_cache.clone()
    _abi.call("ivakv_index_scatter", out.data_ptr(), *out.stride(), idx.data_ptr(), n_idx,
              values.data_ptr(), *values.stride(), batch, n_heads, seq_len, head_dim, code,
              _stream(dev))
    return out
