"""Seeded synthetic workloads for the paged KV hot path (the five BASELINE configs).

Every generator is deterministic in its seed.  Host-side randomness (lengths,
page permutations) comes from ``torch.Generator().manual_seed(seed)`` on the CPU;
bulk K/V/Q values are drawn with a generator on ``device`` (the CPU by default,
so the oracle and the GPU path see identical bits; the bench draws on the GPU).

  C1  paged append then gather, fp32: 4 sequences of {17, 64, 129, 200} tokens,
      8 KV heads, head_dim 64, block 16; block tables are the first pages of a
      seeded permutation of a 64-page pool; K/V ~ N(0, 1).
  C2  paged decode attention, fp16: 32 sequences, 32 query / 8 KV heads,
      head_dim 128, block 16, context ~ U[512, 4096]; Q/K/V ~ N(0,1)/sqrt(128);
      block tables are a seeded page permutation.
  C4  long-context decode, bf16: 4 sequences of 32k/64k/96k/128k tokens, window
      4096 + 4 sinks, 32/8 heads, head_dim 128, K/V ~ N(0, 1).
  C5  ragged churn, fp16: 256 sequences, lengths LogNormal(ln 1024, sigma=1.0)
      capped at 16384 (sigma is not given by the config; 1.0 is stated here),
      block tables fragmented by LIFO free-list reuse (see PagedKVPool).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from .ops import pool_shapes

BLOCK_SIZE = 16


@dataclass
class PagedLayout:
    """Block tables of a batch: sequence b owns pages block_tables[b, :ceil(L_b / bs)]."""
    lengths: List[int]
    block_tables: torch.Tensor  # int32 [B, max_blocks], -1 past each sequence's pages
    num_pages: int
    block_size: int = BLOCK_SIZE

    @property
    def context_lens(self) -> torch.Tensor:
        return torch.tensor(self.lengths, dtype=torch.int32)

    def slots(self, b: int, positions: torch.Tensor) -> torch.Tensor:
        """Slot ids of positions of sequence b."""
        pages = self.block_tables[b].to(torch.int64)[positions // self.block_size]
        return (pages * self.block_size + positions % self.block_size).to(torch.int32)


def permuted_layout(lengths: List[int], num_pages: int, gen: torch.Generator,
                    block_size: int = BLOCK_SIZE, max_blocks: Optional[int] = None) -> PagedLayout:
    """Sequences take consecutive runs of one seeded permutation of the pool's pages."""
    need = [math.ceil(int(n) / block_size) for n in lengths]
    if sum(need) > num_pages:
        raise ValueError(f"{sum(need)} pages needed, pool has {num_pages}")
    perm = torch.randperm(num_pages, generator=gen).to(torch.int32)
    mb = max_blocks if max_blocks is not None else max(need + [1])
    bt = torch.full((len(lengths), mb), -1, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[cur:cur + n]
        cur += n
    return PagedLayout([int(n) for n in lengths], bt, num_pages, block_size)


def _randn(shape, gen_seed: int, device, dtype, scale: float = 1.0) -> torch.Tensor:
    dev = torch.device(device) if device is not None else torch.device("cpu")
    g = torch.Generator(device=dev).manual_seed(gen_seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


def c1_append_gather(seed: int = 0, dtype: torch.dtype = torch.float32, device=None) -> dict:
    """C1: rows of every token of the four sequences plus the slots they go to."""
    lengths = [17, 64, 129, 200]
    hkv, head_dim, num_pages = 8, 64, 64
    gen = torch.Generator().manual_seed(seed)
    layout = permuted_layout(lengths, num_pages, gen)
    n_tok = sum(lengths)
    k_new = _randn((n_tok, hkv, head_dim), seed * 1000 + 1, device, dtype)
    v_new = _randn((n_tok, hkv, head_dim), seed * 1000 + 2, device, dtype)
    slots = torch.cat([layout.slots(b, torch.arange(n)) for b, n in enumerate(lengths)])
    return dict(lengths=lengths, layout=layout, k_new=k_new, v_new=v_new, slot_mapping=slots,
                num_kv_heads=hkv, head_dim=head_dim, num_pages=num_pages, block_size=BLOCK_SIZE)


def random_pools(num_pages: int, hkv: int, head_dim: int, dtype: torch.dtype, seed: int,
                 device=None, scale: float = 1.0):
    """A pool pair filled with N(0, scale^2) values (page contents are i.i.d., so the
    layout of the values inside a page is immaterial)."""
    ks, vs = pool_shapes(num_pages, hkv, head_dim, BLOCK_SIZE, dtype)
    return (_randn(ks, seed * 1000 + 11, device, dtype, scale),
            _randn(vs, seed * 1000 + 12, device, dtype, scale))


def decode_batch(lengths: List[int], num_q_heads: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype, seed: int, device=None, scale: float = 1.0,
                 extra_pages: int = 0, max_blocks: Optional[int] = None) -> dict:
    """Decode inputs: a permuted page layout for ``lengths``, random pools, random q."""
    gen = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(n / BLOCK_SIZE) for n in lengths)
    num_pages = max(need + extra_pages, 1)
    layout = permuted_layout(lengths, num_pages, gen, max_blocks=max_blocks)
    k_pool, v_pool = random_pools(num_pages, num_kv_heads, head_dim, dtype, seed, device, scale)
    q = _randn((len(lengths), num_q_heads, head_dim), seed * 1000 + 13, device, dtype, scale)
    return dict(lengths=list(lengths), layout=layout, k_pool=k_pool, v_pool=v_pool, q=q,
                num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=head_dim)


def prefill_batch(lengths: List[int], chunks: List[int], num_q_heads: int, num_kv_heads: int,
                  head_dim: int, dtype: torch.dtype, seed: int, device=None,
                  scale: float = 1.0) -> dict:
    """Prefill inputs: pools holding ``lengths[b]`` positions of sequence b (the chunk
    already appended) and query rows for its last ``chunks[b]`` positions, packed as
    ``q [sum(chunks), Hq, D]`` with ``query_start`` (int32 ``[B+1]``)."""
    d = decode_batch(lengths, num_q_heads, num_kv_heads, head_dim, dtype, seed, device, scale)
    qs = [0]
    for n in chunks:
        qs.append(qs[-1] + int(n))
    d["q"] = _randn((qs[-1], num_q_heads, head_dim), seed * 1000 + 14, device, dtype, scale)
    d["query_start"] = torch.tensor(qs, dtype=torch.int32)
    d["chunks"] = [int(n) for n in chunks]
    return d


def c2_lengths(seed: int, batch: int = 32, lo: int = 512, hi: int = 4096) -> List[int]:
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()


def c2_decode(seed: int = 0, device=None, batch: int = 32, dtype: torch.dtype = torch.float16) -> dict:
    """C2 at full size: B 32, GQA 32/8, head_dim 128, context U[512, 4096], values N(0,1)/sqrt(128)."""
    lengths = c2_lengths(seed, batch)
    return decode_batch(lengths, 32, 8, 128, dtype, seed, device, scale=1.0 / math.sqrt(128))


C4_LENGTHS = [32 * 1024, 64 * 1024, 96 * 1024, 128 * 1024]
C4_WINDOW = 4096
C4_SINKS = 4


def c4_long_context(seed: int = 0, device=None, lengths: Optional[List[int]] = None,
                    dtype: torch.dtype = torch.bfloat16) -> dict:
    """C4: 4 long sequences, window 4096 + 4 sinks, bf16, K/V ~ N(0, 1)."""
    d = decode_batch(lengths or C4_LENGTHS, 32, 8, 128, dtype, seed, device, scale=1.0)
    d.update(window=C4_WINDOW, n_sink=C4_SINKS)
    return d


def c5_lengths(seed: int, n_seqs: int = 256, median: int = 1024, sigma: float = 1.0,
               cap: int = 16384) -> List[int]:
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(n_seqs, generator=gen, dtype=torch.float64)
    lens = torch.exp(math.log(median) + sigma * z).round().clamp(1, cap)
    return [int(x) for x in lens.tolist()]


class ChurnBatch:
    """Config C5 driver: continuous batching over a PagedKVPool (one layer, fp16,
    GQA 32/8, head_dim 128 by default).

    ``n_seqs`` sequences are live at any time, each with a target length drawn from
    LogNormal(ln median, sigma) capped at ``cap``.  A new sequence is prefilled in
    ``chunk``-token appends; every step appends one decode token to each live
    sequence; a sequence that reaches its target completes, its pages go back to
    the LIFO free list and a new sequence takes its block-table row, reusing those
    pages, so block tables become fragmented.  K/V rows are drawn from a seeded
    device generator; the host keeps the lengths.
    """

    def __init__(self, pool, n_seqs: int = 256, median: int = 1024, sigma: float = 1.0,
                 cap: int = 16384, chunk: int = 512, seed: int = 0, scale: float = 1.0):
        self.pool = pool
        self.n_seqs, self.median, self.sigma, self.cap, self.chunk = n_seqs, median, sigma, cap, chunk
        self.scale = scale
        self.gen = torch.Generator().manual_seed(seed)
        self.dev_gen = torch.Generator(device=pool.device).manual_seed(seed + 1)
        self.ids = []
        self.targets = {}
        self._next = 0
        for _ in range(n_seqs):
            self._start()

    def _draw_length(self) -> int:
        z = torch.randn(1, generator=self.gen, dtype=torch.float64).item()
        return int(max(1, min(self.cap, round(math.exp(math.log(self.median) + self.sigma * z)))))

    def _rows(self, n: int):
        shape = (n, self.pool.num_kv_heads, self.pool.head_dim)
        k = torch.randn(shape, generator=self.dev_gen, device=self.pool.device) * self.scale
        v = torch.randn(shape, generator=self.dev_gen, device=self.pool.device) * self.scale
        return k.to(self.pool.dtype), v.to(self.pool.dtype)

    def _append(self, sid, n: int) -> None:
        from .ops import kv_append
        slots = torch.from_numpy(self.pool.allocate(sid, n)).to(self.pool.device)
        k, v = self._rows(n)
        kv_append(k, v, self.pool.k_pools[0], self.pool.v_pools[0], slots)

    def _start(self) -> None:
        sid = ("c5", self._next)
        self._next += 1
        target = self._draw_length()
        self.pool.add_sequence(sid)
        self.ids.append(sid)
        self.targets[sid] = target
        prompt = max(1, target // 2)
        for off in range(0, prompt, self.chunk):       # prefill-chunk appends
            self._append(sid, min(self.chunk, prompt - off))

    def step(self) -> int:
        """One decode step: one token appended to every live sequence (a single append
        launch), completed sequences freed and replaced by new, chunk-prefilled ones.
        Returns how many sequences completed."""
        import numpy as np
        from .ops import kv_append
        slots = np.concatenate([self.pool.allocate(sid, 1) for sid in self.ids])
        k, v = self._rows(len(self.ids))
        kv_append(k, v, self.pool.k_pools[0], self.pool.v_pools[0],
                  torch.from_numpy(slots).to(self.pool.device))
        finished = [sid for sid in self.ids if self.pool.length(sid) >= self.targets[sid]]
        for sid in finished:
            self.pool.free(sid)
            self.ids.remove(sid)
            del self.targets[sid]
        for _ in finished:
            self._start()
        return len(finished)

    def tables(self):
        """Device block tables and context lengths of the live sequences."""
        return self.pool.device_tables(self.ids)

    def lengths(self):
        return [self.pool.length(s) for s in self.ids]
