"""Paged KV-cache allocator and the ``KVCache`` drop-in built on it.

``PagedKVPool`` owns the device pools of every layer and the host-side page
bookkeeping: a LIFO free list, per-page reference counts (so forked sequences
share full pages), per-sequence block lists and lengths, and the int32 block
tables / context lengths the kernels read.  It replaces the contiguous,
grow-by-copy buffer of ``KVCache`` (src/core/rope_kv.py:71-137): growing a
sequence allocates pages and never copies.

``PagedKVCache`` satisfies the ``KVCache`` duck type used by
``Transformer.forward`` and ``AttentionTorch.forward`` (src/core/rope_kv.py:73-96,
src/core/attention.py:61-73, src/core/transformer.py:200-203,273-279):
``batch_size``, ``n_heads``, ``head_dim``, ``seq_len``, ``device``, ``dtype``,
``k`` / ``v``, ``update``, ``resize``, ``clear``, ``get_slice``.  The reference
threads ONE cache object through every block of a forward
(transformer.py:229-238) and never returns it (:242-255); this cache therefore
keeps one pool per layer, hands them out with a layer cursor (the n-th attention
call of a forward gets layer n) and advances ``seq_len`` in place when the last
layer has appended.

Layout of one layer's pools (X = 16 bytes / element size), see include/ivakv.h:
    k_pool: [num_pages, Hkv, D // X, block_size, X]
    v_pool: [num_pages, Hkv, D, block_size]
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from .ops import FP8, copy_pages, kv_append, kv_gather, pool_shapes, scale_shape


class OutOfPagesError(RuntimeError):
    """The pool's free list cannot satisfy an allocation."""


@dataclass
class _Seq:
    pages: List[int]      # logical page j -> physical page (-1 once released)
    length: int = 0       # tokens written
    reserved: int = 0     # tokens the allocated pages can hold


class PagedKVPool:
    """Pools of ``num_layers`` layers plus the page allocator.

    Sequences are identified by arbitrary hashable ids; each one owns a row of the
    block table.  All page bookkeeping is on the host (numpy); the device mirrors of
    the block table and context lengths are refreshed by :meth:`device_tables`.
    """

    def __init__(self, num_pages: int, num_kv_heads: int, head_dim: int, block_size: int = 16,
                 num_layers: int = 1, dtype: torch.dtype = torch.float16, device="cuda",
                 max_seqs: int = 256, max_blocks_per_seq: Optional[int] = None,
                 allocate_storage: bool = True):
        if num_pages <= 0 or num_kv_heads <= 0 or head_dim <= 0 or block_size <= 0:
            raise ValueError("num_pages, num_kv_heads, head_dim and block_size must be positive")
        self.num_pages = int(num_pages)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.block_size = int(block_size)
        self.num_layers = int(num_layers)
        self.dtype = dtype
        self.device = torch.device(device)
        self.max_seqs = int(max_seqs)
        self.max_blocks = int(max_blocks_per_seq) if max_blocks_per_seq else self.num_pages
        self._free: List[int] = list(range(self.num_pages - 1, -1, -1))  # pop() -> page 0 first
        self._ref = np.zeros(self.num_pages, dtype=np.int32)
        self._seqs: Dict[object, _Seq] = {}
        self._rows: Dict[object, int] = {}
        self._free_rows: List[int] = list(range(self.max_seqs - 1, -1, -1))
        self.block_tables = np.full((self.max_seqs, self.max_blocks), -1, dtype=np.int32)
        self.context_lens = np.zeros(self.max_seqs, dtype=np.int32)
        # bumped by every change of a block-table entry (allocation, release, fork, free,
        # compaction, restore): device copies of the tables are stale once it moves
        self.generation = 0
        self.k_pools: List[torch.Tensor] = []
        self.v_pools: List[torch.Tensor] = []
        # FP8 pools: one fp32 scaling factor per (slot, kv head) and layer
        self.k_scales: List[torch.Tensor] = []
        self.v_scales: List[torch.Tensor] = []
        if allocate_storage:
            ks, vs = pool_shapes(self.num_pages, self.num_kv_heads, self.head_dim,
                                 self.block_size, dtype)
            # one allocation per layer and tensor: 2 * num_layers pools
            for _ in range(self.num_layers):
                self.k_pools.append(torch.zeros(ks, dtype=dtype, device=self.device))
                self.v_pools.append(torch.zeros(vs, dtype=dtype, device=self.device))
                if self.fp8:
                    shape = scale_shape(self.num_pages, self.num_kv_heads, self.block_size)
                    self.k_scales.append(torch.ones(shape, dtype=torch.float32, device=self.device))
                    self.v_scales.append(torch.ones(shape, dtype=torch.float32, device=self.device))

    @property
    def fp8(self) -> bool:
        """Pages hold e4m3fn codes with per-(slot, kv head) scaling factors."""
        return self.dtype == FP8

    def scales(self, layer: int) -> Dict[str, Optional[torch.Tensor]]:
        """``k_scale`` / ``v_scale`` keyword arguments of the ops for one layer."""
        if not self.fp8:
            return {}
        return {"k_scale": self.k_scales[layer], "v_scale": self.v_scales[layer]}

    # ------------------------------------------------------------------ config
    @classmethod
    def from_config(cls, memory_cfg: dict, num_layers: int, num_kv_heads: int, head_dim: int,
                    device="cuda", dtype: torch.dtype = torch.float16, block_size: int = 16,
                    max_seqs: int = 256) -> "PagedKVPool":
        """Pool sized by the ``memory`` block of configs/quant_infer.yaml:50-60:
        ``kv_cache_blocks`` pages, ``kv_cache_size`` tokens per sequence at most,
        ``kv_cache_dtype`` the element type (fp16 / bf16 / fp32, or fp8: e4m3fn codes with
        per-(slot, kv head) scaling factors)."""
        if not memory_cfg.get("paged_kv_cache", True):
            raise ValueError("memory.paged_kv_cache is false: use the contiguous KVCache")
        names = {"fp16": torch.float16, "float16": torch.float16, "bf16": torch.bfloat16,
                 "bfloat16": torch.bfloat16, "fp32": torch.float32, "float32": torch.float32,
                 "fp8": FP8, "fp8_e4m3": FP8, "float8_e4m3fn": FP8}
        kv_dtype = memory_cfg.get("kv_cache_dtype")
        if kv_dtype is not None:
            if str(kv_dtype) not in names:
                raise NotImplementedError(f"kv_cache_dtype {kv_dtype!r} is not supported by the "
                                          "paged KV kernels (fp16, bf16, fp32, fp8)")
            dtype = names[str(kv_dtype)]
        num_pages = int(memory_cfg.get("kv_cache_blocks", 256))
        max_tokens = int(memory_cfg.get("kv_cache_size", num_pages * block_size))
        return cls(num_pages, num_kv_heads, head_dim, block_size, num_layers, dtype, device,
                   max_seqs=max_seqs, max_blocks_per_seq=math.ceil(max_tokens / block_size))

    # ------------------------------------------------------------ page lists
    @property
    def num_free_pages(self) -> int:
        return len(self._free)

    def _take_page(self) -> int:
        if not self._free:
            raise OutOfPagesError(f"no free page left in a pool of {self.num_pages}")
        p = self._free.pop()
        self._ref[p] = 1
        return p

    def _drop_page(self, p: int) -> None:
        if p < 0:
            return
        self._ref[p] -= 1
        if self._ref[p] == 0:
            self._free.append(p)  # LIFO: the next allocation reuses it first

    def _seq(self, seq_id) -> _Seq:
        try:
            return self._seqs[seq_id]
        except KeyError:
            raise KeyError(f"unknown sequence {seq_id!r}") from None

    def _sync_row(self, seq_id) -> None:
        s, row = self._seqs[seq_id], self._rows[seq_id]
        self.generation += 1
        self.block_tables[row, :] = -1
        self.block_tables[row, :len(s.pages)] = s.pages
        self.context_lens[row] = s.length

    def add_sequence(self, seq_id) -> int:
        """Registers an empty sequence; returns its block-table row."""
        if seq_id in self._seqs:
            raise ValueError(f"sequence {seq_id!r} already exists")
        if not self._free_rows:
            raise OutOfPagesError(f"all {self.max_seqs} block-table rows are in use")
        row = self._free_rows.pop()
        self._seqs[seq_id] = _Seq(pages=[])
        self._rows[seq_id] = row
        self._sync_row(seq_id)
        return row

    def has_sequence(self, seq_id) -> bool:
        return seq_id in self._seqs

    def length(self, seq_id) -> int:
        return self._seq(seq_id).length

    def row(self, seq_id) -> int:
        self._seq(seq_id)
        return self._rows[seq_id]

    def pages(self, seq_id) -> List[int]:
        return list(self._seq(seq_id).pages)

    def reserve(self, seq_id, n_tokens: int) -> None:
        """Allocates pages so the sequence can hold ``length + n_tokens`` tokens.
        On exhaustion nothing is allocated and OutOfPagesError is raised."""
        s = self._seq(seq_id)
        if int(n_tokens) < 0:
            raise ValueError(f"n_tokens must be >= 0, got {n_tokens}")
        want = s.length + int(n_tokens)
        need = math.ceil(want / self.block_size) - len(s.pages)
        if need <= 0:
            return
        if len(s.pages) + need > self.max_blocks:
            raise OutOfPagesError(f"sequence {seq_id!r} would need {len(s.pages) + need} pages; "
                                  f"the block table holds {self.max_blocks}")
        if need > len(self._free):
            raise OutOfPagesError(f"sequence {seq_id!r} needs {need} pages, {len(self._free)} free")
        s.pages.extend(self._take_page() for _ in range(need))
        s.reserved = len(s.pages) * self.block_size
        self._sync_row(seq_id)

    def slots(self, seq_id, positions) -> np.ndarray:
        """Slot ids (page * block_size + row) of token positions of a sequence."""
        s = self._seq(seq_id)
        pos = np.asarray(positions, dtype=np.int64)
        if pos.size and (pos.min() < 0 or pos.max() >= len(s.pages) * self.block_size):
            raise IndexError(f"positions outside the pages of sequence {seq_id!r}")
        pages = np.asarray(s.pages, dtype=np.int64)[pos // self.block_size] if pos.size else pos
        if pos.size and (pages < 0).any():
            raise IndexError(f"positions on released pages of sequence {seq_id!r}")
        return (pages * self.block_size + pos % self.block_size).astype(np.int32)

    def allocate(self, seq_id, n_tokens: int) -> np.ndarray:
        """Reserves pages for ``n_tokens`` new tokens, advances the length and returns
        their slot ids (the ``slot_mapping`` of an append).  A negative count raises
        ValueError, as exhaustion raises OutOfPagesError, with nothing changed."""
        s = self._seq(seq_id)
        self.reserve(seq_id, n_tokens)
        start = s.length
        s.length += int(n_tokens)
        self.context_lens[self._rows[seq_id]] = s.length
        return self.slots(seq_id, np.arange(start, s.length))

    def free(self, seq_id) -> None:
        """Returns the sequence's pages to the free list (shared pages stay until their
        last owner frees them) and releases its block-table row."""
        s = self._seq(seq_id)
        for p in reversed(s.pages):
            self._drop_page(p)
        row = self._rows.pop(seq_id)
        del self._seqs[seq_id]
        self.generation += 1
        self.block_tables[row, :] = -1
        self.context_lens[row] = 0
        self._free_rows.append(row)

    def fork(self, src_id, dst_id) -> None:
        """New sequence ``dst_id`` with the content of ``src_id``: full pages are shared
        (reference counted), the partial last page is copied into a fresh page."""
        s = self._seq(src_id)
        self.add_sequence(dst_id)
        d = self._seqs[dst_id]
        full = s.length // self.block_size
        try:
            for p in s.pages[:full]:
                if p >= 0:
                    self._ref[p] += 1
                d.pages.append(p)
            if s.length % self.block_size:
                src_page = s.pages[full]
                new_page = self._take_page()
                d.pages.append(new_page)
                for t in self.k_pools + self.v_pools + self.k_scales + self.v_scales:
                    t[new_page].copy_(t[src_page])
        except OutOfPagesError:
            self.free(dst_id)
            raise
        d.length = s.length
        d.reserved = len(d.pages) * self.block_size
        self._sync_row(dst_id)

    def release_outside_window(self, seq_id, window: int, n_sink: int = 0) -> int:
        """Frees the pages of a sequence that hold no position a decode query can still
        see: with length L, visible positions are [0, n_sink) and [L - window, L) (the
        window/sink union of the decode kernel).  Their block-table entries become -1.
        Positions only move forward, so a released page never becomes visible again.
        Returns the number of pages released."""
        s = self._seq(seq_id)
        if window <= 0:
            return 0
        first_visible = max(s.length - int(window), 0)
        sink_pages = math.ceil(max(int(n_sink), 0) / self.block_size)
        released = 0
        for j in range(sink_pages, min(first_visible // self.block_size, len(s.pages))):
            if s.pages[j] >= 0:
                self._drop_page(s.pages[j])
                s.pages[j] = -1
                released += 1
        if released:
            self._sync_row(seq_id)
        return released

    # ------------------------------------------------------------ compaction
    def compaction_moves(self) -> Tuple[List[int], List[int]]:
        """(src, dst) page moves that pack the referenced pages into ids [0, n_used):
        every referenced page at or above n_used goes to a free id below it, in
        ascending order of both.  The two sets are disjoint."""
        n_used = int((self._ref > 0).sum())
        src = [int(p) for p in np.nonzero(self._ref > 0)[0] if p >= n_used]
        dst = [int(p) for p in range(n_used) if self._ref[p] == 0]
        return src, dst

    def compact(self) -> int:
        """Packs the live pages into the lowest page ids, moving their contents (every
        layer, and the FP8 scaling factors) with ivakv_copy_pages and renumbering the
        block tables; the free list becomes the contiguous tail [n_used, num_pages).
        The paged counterpart of kv_compact_triton (src/kernels_t/kv_ops_triton.py:
        68-92,159-181): after it, the pool holds no gaps below its last live page.
        Device copies of block tables taken earlier are stale.  Returns the pages moved."""
        src, dst = self.compaction_moves()
        if not src:
            return 0
        if self.k_pools:
            s_t = torch.tensor(src, dtype=torch.int32).to(self.device)
            d_t = torch.tensor(dst, dtype=torch.int32).to(self.device)
            for layer in range(self.num_layers):
                copy_pages(self.k_pools[layer], self.v_pools[layer], s_t, d_t,
                           **self.scales(layer))
        remap = np.arange(self.num_pages)
        remap[src] = dst
        for seq_id, seq in self._seqs.items():
            seq.pages = [int(remap[p]) if p >= 0 else p for p in seq.pages]
            self._sync_row(seq_id)
        self._ref[dst] = self._ref[src]
        self._ref[src] = 0
        n_used = int((self._ref > 0).sum())
        self._free = list(range(self.num_pages - 1, n_used - 1, -1))  # pop() -> n_used first
        return len(src)

    # --------------------------------------------------------------- batches
    def tables(self, seq_ids: Sequence) -> Tuple[np.ndarray, np.ndarray]:
        """(block_tables [B, max_blocks], context_lens [B]) of a batch, host int32."""
        rows = [self.row(s) for s in seq_ids]
        used = max((len(self._seqs[s].pages) for s in seq_ids), default=0)
        width = max(used, 1)
        return (np.ascontiguousarray(self.block_tables[rows, :width]),
                np.ascontiguousarray(self.context_lens[rows]))

    def device_tables(self, seq_ids: Sequence) -> Tuple[torch.Tensor, torch.Tensor]:
        bt, ctx = self.tables(seq_ids)
        return (torch.from_numpy(bt).to(self.device, non_blocking=True),
                torch.from_numpy(ctx).to(self.device, non_blocking=True))

    # ------------------------------------------------------------ persistence
    def state_dict(self) -> dict:
        """Allocator state (not the pool contents): free list, refcounts, sequences."""
        return {"free": list(self._free), "ref": self._ref.copy(),
                "seqs": {k: (list(v.pages), v.length) for k, v in self._seqs.items()},
                "rows": dict(self._rows), "free_rows": list(self._free_rows),
                "geometry": (self.num_pages, self.num_kv_heads, self.head_dim, self.block_size,
                             self.num_layers, self.max_seqs, self.max_blocks)}

    def load_state_dict(self, state: dict) -> None:
        geo = (self.num_pages, self.num_kv_heads, self.head_dim, self.block_size,
               self.num_layers, self.max_seqs, self.max_blocks)
        if tuple(state["geometry"]) != geo:
            raise ValueError(f"allocator state is for geometry {state['geometry']}, pool is {geo}")
        self._free = list(state["free"])
        self._ref = np.array(state["ref"], dtype=np.int32)
        self._rows = dict(state["rows"])
        self._free_rows = list(state["free_rows"])
        self._seqs = {k: _Seq(pages=list(p), length=int(n), reserved=len(p) * self.block_size)
                      for k, (p, n) in state["seqs"].items()}
        self.generation += 1
        self.block_tables[:] = -1
        self.context_lens[:] = 0
        for k in self._seqs:
            self._sync_row(k)


@dataclass
class LayerView:
    """What one attention layer of one forward gets from a PagedKVCache."""
    layer: int
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    slot_mapping: torch.Tensor   # int32 [B * T], token-major (b, t)
    block_tables: torch.Tensor   # int32 [B, max_blocks]
    context_lens: torch.Tensor   # int32 [B], lengths after this forward's append
    start: int                   # position of the first new token
    new_tokens: int              # T
    scales: Dict[str, torch.Tensor] = field(default_factory=dict)  # FP8: k_scale / v_scale


class PagedKVCache:
    """``KVCache`` (src/core/rope_kv.py:71-137) over a PagedKVPool, for every layer.

    ``n_heads`` is the number of KV heads.  All sequences of the batch advance together
    by the tokens of each forward, as in ``KVCache`` (one ``seq_len`` for the batch).
    ``seq_len > 0`` at construction starts every sequence with that many zero rows,
    as ``KVCache`` does.
    """

    def __init__(self, batch_size: int, n_heads: int, head_dim: int, seq_len: int = 0,
                 device=None, dtype: torch.dtype = torch.float16, *, num_layers: int = 1,
                 block_size: int = 16, max_seq_len: int = 4096, num_pages: Optional[int] = None,
                 pool: Optional[PagedKVPool] = None, compute_dtype: Optional[torch.dtype] = None,
                 release_window: bool = True):
        self.batch_size = int(batch_size)
        # sliding-window attention: pages no later query can see go back to the pool
        # after each forward (release_window), the sink pages stay resident
        self.window_release = bool(release_window)
        self._window: Optional[Tuple[int, int]] = None     # (window, n_sink) noted this forward
        self._released: Optional[Tuple[int, int]] = None   # strictest policy applied so far
        self.n_heads = int(n_heads)
        self.head_dim = int(head_dim)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.dtype = dtype
        # FP8 pages: rows written from and read back as float16 unless told otherwise
        self.compute_dtype = compute_dtype or (torch.float16 if dtype == FP8 else dtype)
        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        if pool is None:
            per_seq = math.ceil(max(int(max_seq_len), int(seq_len), 1) / block_size)
            pages = num_pages if num_pages is not None else per_seq * self.batch_size
            pool = PagedKVPool(pages, self.n_heads, self.head_dim, block_size, self.num_layers,
                               dtype, self.device, max_seqs=max(self.batch_size, 1),
                               max_blocks_per_seq=per_seq)
        elif (pool.num_kv_heads, pool.head_dim, pool.num_layers) != (self.n_heads, self.head_dim,
                                                                     self.num_layers):
            raise ValueError("pool geometry does not match the cache")
        self.pool = pool
        self.seq_ids = list(self._new_ids())
        for s in self.seq_ids:
            pool.add_sequence(s)
        self.seq_len = 0
        self._cursor = 0
        self._view: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int]] = None
        self._bt_dev: Optional[torch.Tensor] = None
        self._bt_gen = -1      # pool generation the device block table was copied at
        self._static: Optional[dict] = None
        self._positions: Optional[torch.Tensor] = None
        if seq_len > 0:
            z = torch.zeros(self.batch_size, self.n_heads, int(seq_len), self.head_dim,
                            dtype=self.compute_dtype, device=self.device)
            for layer in range(self.num_layers):
                self._cursor = layer
                self._append_all(z, z, layer_only=layer, commit=layer == self.num_layers - 1)
            self._cursor = 0

    _next_id = 0

    def _new_ids(self):
        for _ in range(self.batch_size):
            PagedKVCache._next_id += 1
            yield ("cache", PagedKVCache._next_id)

    # ----------------------------------------------------------- duck type
    @property
    def current_layer(self) -> int:
        return self._cursor

    def select_layer(self, layer: int) -> None:
        """Points ``k``, ``v``, ``get_slice`` and ``update`` at one layer (direct use of the
        KVCache API; a model forward moves the cursor itself)."""
        if not 0 <= layer < self.num_layers:
            raise IndexError(f"layer {layer} of a {self.num_layers}-layer cache")
        if self._view is not None:
            raise RuntimeError("a forward is in progress on this cache")
        self._cursor = int(layer)

    def layer_kv(self, layer: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Contiguous [B, Hkv, seq_len, D] K and V of one layer (gathered, a copy)."""
        bt, ctx = self._tables()
        return kv_gather(self.pool.k_pools[layer], self.pool.v_pools[layer], bt, ctx,
                         out_len=self.seq_len, **self._gather_kw(layer))

    def _gather_kw(self, layer: int) -> dict:
        kw = dict(self.pool.scales(layer))
        if kw:  # FP8 pages read back in the cache's compute dtype
            kw["out_dtype"] = self.compute_dtype
        return kw

    @property
    def k(self) -> torch.Tensor:
        return self.layer_kv(self._cursor)[0]

    @property
    def v(self) -> torch.Tensor:
        return self.layer_kv(self._cursor)[1]

    def get_slice(self, start: int, end: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Rows [start, end) of the current layer (a copy; KVCache returns a view)."""
        k, v = self.layer_kv(self._cursor)
        return k[:, :, start:end], v[:, :, start:end]

    def resize(self, new_seq_len: int) -> None:
        """Reserves pages for ``new_seq_len`` tokens per sequence (no copy, no length change)."""
        for s in self.seq_ids:
            self.pool.reserve(s, max(int(new_seq_len) - self.pool.length(s), 0))

    def clear(self) -> None:
        """Zero-fills the cached rows of every layer (KVCache.clear, rope_kv.py:132-134)."""
        for k, v in zip(self.pool.k_pools, self.pool.v_pools):
            pages = [p for s in self.seq_ids for p in self.pool.pages(s) if p >= 0]
            if pages:
                idx = torch.tensor(pages, device=k.device)
                if self.pool.fp8:  # code 0 is +0.0 whatever the scaling factor
                    k, v = k.view(torch.uint8), v.view(torch.uint8)
                k.index_fill_(0, idx, 0)
                v.index_fill_(0, idx, 0)

    def update(self, new_k: torch.Tensor, new_v: torch.Tensor, start_pos: int) -> None:
        """KVCache.update (rope_kv.py:98-110) on the current layer: rows of ``new_k`` /
        ``new_v`` ([B, Hkv, T, D]) land at positions [start_pos, start_pos + T).
        Positions past the current length extend every sequence (pages are allocated);
        when the pool cannot hold the whole batch's growth, OutOfPagesError is raised
        before any sequence grows."""
        t = new_k.shape[2]
        end = int(start_pos) + t
        layer = self._cursor
        bs = self.pool.block_size
        need = [max(0, -(-end // bs) - len(self.pool.pages(s))) for s in self.seq_ids]
        if sum(need) > self.pool.num_free_pages:
            raise OutOfPagesError(f"the batch needs {sum(need)} pages, "
                                  f"{self.pool.num_free_pages} free")
        for s in self.seq_ids:
            grow = end - self.pool.length(s)
            if grow > 0:
                self.pool.allocate(s, grow)
        slots = np.concatenate([self.pool.slots(s, np.arange(start_pos, end)) for s in self.seq_ids])
        rows_k = new_k.permute(0, 2, 1, 3).reshape(-1, self.n_heads, self.head_dim)
        rows_v = new_v.permute(0, 2, 1, 3).reshape(-1, self.n_heads, self.head_dim)
        kv_append(rows_k, rows_v, self.pool.k_pools[layer], self.pool.v_pools[layer],
                  torch.from_numpy(slots).to(self.device), **self.pool.scales(layer))
        self.seq_len = max(self.seq_len, end)
        self._bt_gen = -1

    def free(self) -> None:
        """Returns every page of this cache's sequences to the pool."""
        for s in self.seq_ids:
            if self.pool.has_sequence(s):
                self.pool.free(s)

    # ------------------------------------------------------ window release
    @property
    def window_policy(self) -> Optional[Tuple[int, int]]:
        """(window, n_sink) the current forward attends with, or None (full context)."""
        return self._window

    def note_window(self, window: Optional[int], n_sink: int = 0) -> None:
        """Records the sliding window and attention sinks the forward about to run attends
        with (decode and prefill queries at position p see [0, n_sink) and
        [p - window + 1, p]; the decode kernels' union, src/core/attention.py:83-93,
        115-148).  Once pages outside a window were released, a forward may only attend
        to what stayed resident: a window no larger and sinks within the kept sink pages;
        anything else raises ValueError."""
        w = int(window) if window is not None and int(window) > 0 else 0
        ns = max(int(n_sink), 0) if w else 0
        if self._released is not None:
            rw, rs = self._released
            kept_sinks = math.ceil(rs / self.block_size) * self.block_size
            if w == 0 or w > rw or ns > kept_sinks:
                raise ValueError(
                    f"pages outside a window of {rw} tokens (+ {rs} sink tokens) were released; "
                    f"a forward with window {w or None} and {ns} sinks would read them "
                    "(construct the cache with release_window=False to keep every page)")
        self._window = (w, ns) if w else None

    def release_window(self) -> int:
        """Returns to the pool the pages that no later query of this cache can see under
        the noted window (:meth:`PagedKVPool.release_outside_window`): with length L only
        the sink pages and [L - window, L) stay resident, so a long sequence holds about
        window + sinks tokens per layer.  Released positions read back as zeros through
        ``k`` / ``v`` / ``get_slice``.  A no-op without a window, with
        ``release_window=False``, or in static decode (its captured graph holds the block
        table; :meth:`end_static_decode` releases).  Returns the pages released."""
        if self._window is None or not self.window_release or self._static is not None:
            return 0
        w, ns = self._window
        n = sum(self.pool.release_outside_window(s, w, ns) for s in self.seq_ids)
        if n:
            rw, rs = self._released if self._released is not None else (w, ns)
            self._released = (min(rw, w), min(rs, ns))
            self._bt_gen = -1
        return n

    def resident_pages(self) -> int:
        """Pages this cache's sequences hold (per layer)."""
        return sum(1 for s in self.seq_ids for p in self.pool.pages(s) if p >= 0)

    # ------------------------------------------------------- layer cursor
    def _tables(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Device block table (copied again only when the pool's tables changed since the
        last copy) and context lengths of this cache's sequences."""
        bt, ctx = self.pool.tables(self.seq_ids)
        gen = self.pool.generation
        if self._bt_dev is None or self._bt_gen != gen or self._bt_dev.shape != bt.shape:
            self._bt_dev = torch.from_numpy(bt).to(self.device)
            self._bt_gen = gen
        return self._bt_dev, torch.from_numpy(ctx).to(self.device)

    # ------------------------------------------------------ static decode
    @property
    def static(self) -> bool:
        return self._static is not None

    def begin_static_decode(self, steps: int) -> None:
        """Switches to single-token steps whose bookkeeping runs on the device, so a
        whole decode step can be captured in a HIP graph and replayed.  Pages for
        ``steps`` more tokens per sequence are reserved now; each step then derives
        the new token's slot from the (fixed) block table and the device context
        lengths, and advances those lengths, with device ops only.  The host-side
        ``seq_len`` is advanced by :meth:`advance_host` (once per replay);
        :meth:`end_static_decode` writes the lengths back to the pool."""
        if self._view is not None or self._cursor != 0:
            raise RuntimeError("a forward is in progress on this cache")
        self.resize(self.seq_len + int(steps))
        bt, ctx = self.pool.tables(self.seq_ids)
        self._static = {
            "bt": torch.from_numpy(bt).to(self.device),
            "ctx": torch.from_numpy(ctx).to(self.device),
            "slot": torch.empty(self.batch_size, dtype=torch.int32, device=self.device),
            "pos": torch.empty(self.batch_size, 1, dtype=torch.int64, device=self.device),
            "rope_pos": torch.empty(self.batch_size, dtype=torch.int32, device=self.device),
            "limit": self.seq_len + int(steps),
        }
        self._static["pos"].copy_(self._static["ctx"].view(-1, 1))

    def device_positions(self) -> torch.Tensor:
        """int64 [B, 1] positions of the next token (static decode), on the device."""
        st = self._static
        st["pos"].copy_(st["ctx"].view(-1, 1))
        return st["pos"]

    def advance_host(self, steps: int = 1) -> None:
        """Host-side length bookkeeping for ``steps`` replayed static decode steps."""
        self.seq_len += int(steps)
        if self.seq_len > self._static["limit"]:
            raise RuntimeError("static decode ran past the reserved pages")

    def end_static_decode(self) -> None:
        """Leaves static decode: the pool's lengths catch up with ``seq_len``."""
        if self._static is None:
            return
        for s in self.seq_ids:
            grow = self.seq_len - self.pool.length(s)
            if grow > 0:
                self.pool.allocate(s, grow)
        self._static = None
        self._bt_gen = -1
        self.release_window()

    def _static_step(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int]:
        st = self._static
        ctx = st["ctx"]
        page = st["bt"].gather(1, torch.div(ctx, self.block_size, rounding_mode="floor")
                               .long().view(-1, 1)).view(-1)
        st["slot"].copy_(page * self.block_size + ctx % self.block_size)
        ctx.add_(1)
        return st["slot"], st["bt"], ctx, self.seq_len, 1

    def token_positions(self, t: int) -> torch.Tensor:
        """Absolute positions of this forward's ``t`` new tokens per sequence, int32
        ``[B * t]`` token-major on the device.  Computed at the first layer and reused by
        the others; in static decode read from the device-side lengths (graph-safe)."""
        if self._cursor == 0 or self._positions is None:
            if self._static is not None:
                buf = self._static["rope_pos"]
                buf.copy_(self._static["ctx"])
                self._positions = buf
            else:
                self._positions = torch.arange(self.seq_len, self.seq_len + int(t), dtype=torch.int32,
                                               device=self.device).repeat(self.batch_size)
        return self._positions

    def layer_step(self, k_rows: torch.Tensor, v_rows: torch.Tensor,
                   append: bool = True, rope_positions: Optional[torch.Tensor] = None,
                   rope_theta: float = 10000.0) -> LayerView:
        """Appends the new tokens' K/V rows ([B, T, Hkv, D]) of the layer at the cursor and
        returns that layer's view.  The first call of a forward allocates the pages of
        the T new tokens of every sequence; the call of the last layer advances
        ``seq_len`` by T and rewinds the cursor.  ``append=False`` allocates and
        advances the same way but leaves writing the rows to the caller (the fused
        decode op writes them itself)."""
        b, t = k_rows.shape[0], k_rows.shape[1]
        if b != self.batch_size:
            raise ValueError(f"batch {b} != cache batch {self.batch_size}")
        if self._cursor == 0 and self._static is not None:
            if t != 1:
                raise ValueError("static decode appends one token per step")
            self._view = self._static_step()
        elif self._cursor == 0:
            start = self.seq_len
            slots = np.concatenate([self.pool.allocate(s, t) for s in self.seq_ids])
            slot_dev = torch.from_numpy(slots).to(self.device, non_blocking=True)
            bt, ctx = self._tables()
            self._view = (slot_dev, bt, ctx, start, t)
        elif self._view is None or self._view[4] != t:
            raise RuntimeError("layer cursor out of step: every layer of a forward must append "
                               "the same tokens")
        slot_dev, bt, ctx, start, t = self._view
        layer = self._cursor
        if append:
            rope = {} if rope_positions is None else {"rope_positions": rope_positions,
                                                      "rope_theta": rope_theta}
            kv_append(k_rows.reshape(b * t, self.n_heads, self.head_dim),
                      v_rows.reshape(b * t, self.n_heads, self.head_dim),
                      self.pool.k_pools[layer], self.pool.v_pools[layer], slot_dev,
                      **self.pool.scales(layer), **rope)
        view = LayerView(layer, self.pool.k_pools[layer], self.pool.v_pools[layer], slot_dev, bt,
                         ctx, start, t, self.pool.scales(layer))
        self._cursor += 1
        if self._cursor == self.num_layers:
            self._cursor = 0
            if self._static is None:
                self.seq_len = start + t
            self._view = None
        return view

    def reset_cursor(self) -> None:
        """Rewinds the layer cursor after a forward that did not reach the last layer
        (the tokens it allocated stay allocated and count as written)."""
        if self._view is not None:
            self.seq_len = self._view[3] + self._view[4]
        self._cursor = 0
        self._view = None

    def _append_all(self, k, v, layer_only: int, commit: bool) -> None:
        """Construction helper: writes [B, Hkv, T, D] rows into one layer at positions 0..T-1."""
        t = k.shape[2]
        if layer_only == 0:
            for s in self.seq_ids:
                self.pool.allocate(s, t)
        slots = np.concatenate([self.pool.slots(s, np.arange(t)) for s in self.seq_ids])
        kv_append(k.permute(0, 2, 1, 3).reshape(-1, self.n_heads, self.head_dim),
                  v.permute(0, 2, 1, 3).reshape(-1, self.n_heads, self.head_dim),
                  self.pool.k_pools[layer_only], self.pool.v_pools[layer_only],
                  torch.from_numpy(slots).to(self.device), **self.pool.scales(layer_only))
        if commit:
            self.seq_len = t


def create_kv_cache(batch_size: int, n_heads: int, head_dim: int, seq_len: int,
                    device=None, dtype: torch.dtype = torch.float16, **kwargs) -> PagedKVCache:
    """The paged counterpart of the reference's factory ``create_kv_cache(batch_size,
    n_heads, head_dim, seq_len, device, dtype=torch.float16)`` (src/core/rope_kv.py:165-173):
    same arguments and meaning (``seq_len`` zero rows per sequence to start with, as
    ``KVCache`` allocates), returning a :class:`PagedKVCache`.  Keyword arguments go to
    the PagedKVCache constructor (``num_layers``, ``max_seq_len``, ``num_pages``, ``pool``,
    ``block_size``, ``compute_dtype``, ``release_window``); ``max_seq_len`` defaults to
    ``seq_len`` (at least one page), and the pool grows no further than the pages it
    reserves for that."""
    kwargs.setdefault("max_seq_len", max(int(seq_len), 1))
    return PagedKVCache(batch_size, n_heads, head_dim, seq_len, device, dtype, **kwargs)

