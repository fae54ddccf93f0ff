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
  C5  ragged churn, fp16: 256 live sequences, total lengths LogNormal(ln 1024,
      sigma=1.0) capped at 16384 (sigma is not given by the config; 1.0 is stated
      here), the last Uniform{1..256} tokens decoded one per step after 512-token
      prefill chunks, completed sequences replaced; block tables fragmented by LIFO
      free-list reuse (see PagedKVPool and ChurnBatch).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
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


def window_layout(lengths: List[int], window: int, n_sink: int, gen: torch.Generator,
                  block_size: int = BLOCK_SIZE) -> PagedLayout:
    """The block tables a sliding-window cache holds once the pages outside the window and
    the sinks are released (PagedKVPool.release_outside_window): sequence b of length L
    keeps the sink pages [0, ceil(n_sink / bs)) and the pages from (L - window) // bs on;
    the entries between are -1.  The kept pages are a seeded permutation of a pool of
    exactly that many pages."""
    sink_pages = math.ceil(max(int(n_sink), 0) / block_size)
    keep = []
    for n in lengths:
        n_log = math.ceil(int(n) / block_size)
        first = max((int(n) - int(window)) // block_size, sink_pages) if window > 0 else sink_pages
        keep.append(list(range(min(sink_pages, n_log))) + list(range(first, n_log)))
    num_pages = max(sum(len(k) for k in keep), 1)
    perm = torch.randperm(num_pages, generator=gen).to(torch.int32)
    mb = max([math.ceil(int(n) / block_size) for n in lengths] + [1])
    bt = torch.full((len(lengths), mb), -1, dtype=torch.int32)
    cur = 0
    for b, k in enumerate(keep):
        bt[b, k] = perm[cur:cur + len(k)]
        cur += len(k)
    return PagedLayout([int(n) for n in lengths], bt, num_pages, block_size)


def c4_long_context(seed: int = 0, device=None, lengths: Optional[List[int]] = None,
                    dtype: torch.dtype = torch.bfloat16, resident_window: bool = False) -> dict:
    """C4: 4 long sequences, window 4096 + 4 sinks, bf16, K/V ~ N(0, 1).  With
    ``resident_window`` the pool holds only the pages a sliding-window cache keeps
    resident (window_layout: the sink pages and the window's), as PagedKVCache does after
    each forward; otherwise every page of every context."""
    lengths = lengths or C4_LENGTHS
    if not resident_window:
        d = decode_batch(lengths, 32, 8, 128, dtype, seed, device, scale=1.0)
    else:
        gen = torch.Generator().manual_seed(seed)
        layout = window_layout(lengths, C4_WINDOW, C4_SINKS, gen)
        k_pool, v_pool = random_pools(layout.num_pages, 8, 128, dtype, seed, device, 1.0)
        q = _randn((len(lengths), 32, 128), seed * 1000 + 13, device, dtype, 1.0)
        d = dict(lengths=list(lengths), layout=layout, k_pool=k_pool, v_pool=v_pool, q=q,
                 num_q_heads=32, num_kv_heads=8, head_dim=128)
    d.update(window=C4_WINDOW, n_sink=C4_SINKS)
    return d


def c5_lengths(seed: int, n_seqs: int = 256, median: int = 1024, sigma: float = 1.0,
               cap: int = 16384) -> List[int]:
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(n_seqs, generator=gen, dtype=torch.float64)
    lens = torch.exp(math.log(median) + sigma * z).round().clamp(1, cap)
    return [int(x) for x in lens.tolist()]


class ChurnBatch:
    """Config C5 driver: continuous batching over a PagedKVPool (one layer).

    Every live sequence has a total length T ~ LogNormal(ln median, sigma) capped at
    ``cap``.  Its last G ~ Uniform{1, ..., gen_max} tokens (at most T - 1) are generated
    one per step; the first P = T - G are its prompt, appended ``chunk`` tokens per step
    (chunked prefill).  A sequence whose length reaches T completes: its pages go back
    to the pool's LIFO free list and a new sequence (length 0, in prefill) takes its
    block-table row and, through the free list, its pages, so tables fragment.  At
    construction every sequence is placed at a uniformly random step of its lifetime
    and the rows it would hold by then are written: the batch starts in steady state,
    and prefill chunks, decode tokens and completions occur on (almost) every step.

    :meth:`plan_step` does the host bookkeeping of one step (allocates its slots) and
    returns what the step appends; :meth:`finish_step` retires completed sequences.
    K/V rows come from a seeded device generator.
    """

    def __init__(self, pool, n_seqs: int = 256, median: int = 1024, sigma: float = 1.0,
                 cap: int = 16384, chunk: int = 512, gen_max: int = 256, seed: int = 0,
                 scale: float = 1.0, fill: bool = True):
        self.pool = pool
        self.n_seqs, self.median, self.sigma, self.cap = n_seqs, median, sigma, cap
        self.chunk, self.gen_max, self.scale = chunk, gen_max, scale
        self.gen = torch.Generator().manual_seed(seed)
        self.dev_gen = (torch.Generator(device=pool.device).manual_seed(seed + 1)
                        if fill else None)
        self.ids: List = []
        self.target: dict = {}
        self.prompt: dict = {}
        self.completed = 0
        self._next = 0
        starts = []
        for _ in range(n_seqs):
            sid = self._start()
            t, p = self.target[sid], self.prompt[sid]
            n_pre = math.ceil(p / chunk)
            life = n_pre + (t - p)
            s_ = int(torch.randint(0, life, (1,), generator=self.gen))
            n0 = min(s_ * chunk, p) if s_ < n_pre else p + (s_ - n_pre)
            starts.append((sid, n0))
        # The rows each sequence holds by now, allocated a page at a time in rounds over
        # the batch (in a shuffled order each round), as their growth would have
        # interleaved: the tables are fragmented from the first step.
        left = {sid: n0 for sid, n0 in starts}
        got = {sid: [] for sid, _ in starts}
        while left:
            order = list(left)
            perm = torch.randperm(len(order), generator=self.gen).tolist()
            for j in perm:
                sid = order[j]
                n = min(self.pool.block_size, left[sid])
                got[sid].append(self.pool.allocate(sid, n))
                left[sid] -= n
                if left[sid] == 0:
                    del left[sid]
        if fill:
            self._write(np.concatenate([np.concatenate(v) for v in got.values() if v]))

    def _draw(self):
        z = torch.randn(1, generator=self.gen, dtype=torch.float64).item()
        t = int(max(2, min(self.cap, round(math.exp(math.log(self.median) + self.sigma * z)))))
        g = int(torch.randint(1, self.gen_max + 1, (1,), generator=self.gen))
        return t, t - min(g, t - 1)

    def _start(self):
        sid = ("c5", self._next)
        self._next += 1
        self.target[sid], self.prompt[sid] = self._draw()
        self.pool.add_sequence(sid)
        self.ids.append(sid)
        return sid

    def _rows(self, n: int, heads: int):
        shape = (n, heads, self.pool.head_dim)
        return (torch.randn(shape, generator=self.dev_gen, device=self.pool.device)
                * self.scale).to(self.pool.dtype)

    def _write(self, slots) -> None:
        from .ops import kv_append
        for lo in range(0, len(slots), 1 << 16):
            sl = torch.from_numpy(np.ascontiguousarray(slots[lo:lo + (1 << 16)])).to(self.pool.device)
            hkv = self.pool.num_kv_heads
            kv_append(self._rows(len(sl), hkv), self._rows(len(sl), hkv), self.pool.k_pools[0],
                      self.pool.v_pools[0], sl)

    def plan_step(self) -> dict:
        """Allocates this step's slots: a chunk of up to ``chunk`` prompt tokens for every
        sequence still in prefill, one token for every sequence in decode.  Returns host
        lists: ``prefill`` [(sid, n)], ``prefill_slots`` (int32, the chunks' slots in
        order), ``decode`` [sid] (their new token is the last position of the updated
        lengths)."""
        prefill, pre_slots, decode = [], [], []
        for sid in self.ids:
            n_now, p = self.pool.length(sid), self.prompt[sid]
            if n_now < p:
                n = min(self.chunk, p - n_now)
                pre_slots.append(self.pool.allocate(sid, n))
                prefill.append((sid, n))
            else:
                self.pool.allocate(sid, 1)
                decode.append(sid)
        slots = np.concatenate(pre_slots) if pre_slots else np.zeros(0, dtype=np.int32)
        return {"prefill": prefill, "prefill_slots": slots.astype(np.int32), "decode": decode}

    def finish_step(self) -> int:
        """Retires the sequences that reached their length and starts new ones in their
        rows; returns how many completed."""
        done = [sid for sid in self.ids if self.pool.length(sid) >= self.target[sid]]
        for sid in done:
            self.pool.free(sid)
            self.ids.remove(sid)
            del self.target[sid], self.prompt[sid]
        for _ in done:
            self._start()
        self.completed += len(done)
        return len(done)

    def lengths(self, ids=None) -> List[int]:
        return [self.pool.length(s) for s in (self.ids if ids is None else ids)]

    def tables(self, ids=None):
        """Device block tables and context lengths of ``ids`` (default: all live)."""
        return self.pool.device_tables(self.ids if ids is None else ids)

    def lognormal_mean(self) -> float:
        """Mean of the stated length distribution (LogNormal(ln median, sigma) capped at
        cap), by quadrature of the capped distribution."""
        mu, s = math.log(self.median), self.sigma
        z = torch.linspace(-8, 8, 20001, dtype=torch.float64)
        w = torch.exp(-0.5 * z * z)
        x = torch.exp(mu + s * z).clamp(max=self.cap)
        return float((w * x).sum() / w.sum())
