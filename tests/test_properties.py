"""Property-based tests (hypothesis) on the CPU: the page pool's bookkeeping under random
sequences of operations, and the oracle's invariants on random shapes.

Pool (PagedKVPool without device storage): after every operation, reference counts
equal the number of block-table entries naming each page; the free list and the
referenced pages partition the pool; block tables and context lengths mirror the
sequences; a page two sequences share sits at the same logical index of both, where
both hold a full page; window release leaves every still-visible position on a page;
compaction renumbers pages without changing which entries share a page.

Oracle (oracle/paged_kv.py): gather(append(rows)) returns the rows bit for bit;
relabelling physical pages (pool contents and table ids together) leaves gather and
decode attention bit-identical; a window at least as long as the context, or one
covered by sinks, equals no window; decode attention is linear in V; scaling q by s
and the softmax scale by 1/s changes nothing; every prefill row equals the decode
oracle at its position.
"""
from __future__ import annotations

import math
from importlib import import_module

import numpy as np
import pytest
from hypothesis import HealthCheck, assume, given, settings
from hypothesis import strategies as st
from hypothesis.stateful import (Bundle, RuleBasedStateMachine, consumes, invariant, precondition,
                                 rule)

from oracle import paged_kv as orc

BS = 16
NUM_PAGES = 48
MAX_SEQS = 10


def _pool_module():
    import iva_amd  # noqa: F401  (the package alias conftest installs)
    return import_module("iva_amd.paged_cache")


@pytest.fixture(autouse=True)
def _package(iva):
    return iva


class PoolMachine(RuleBasedStateMachine):
    seqs = Bundle("seqs")

    def __init__(self):
        super().__init__()
        pc = _pool_module()
        self.pc = pc
        self.pool = pc.PagedKVPool(NUM_PAGES, 2, 64, BS, allocate_storage=False, device="cpu",
                                   max_seqs=MAX_SEQS, max_blocks_per_seq=24)
        self.n = 0
        self.live = set()

    def _new_id(self):
        self.n += 1
        return ("s", self.n)

    @precondition(lambda self: len(self.live) < MAX_SEQS)
    @rule(target=seqs)
    def add(self):
        sid = self._new_id()
        self.pool.add_sequence(sid)
        self.live.add(sid)
        return sid

    @rule(sid=seqs, n=st.integers(0, 70))
    def allocate(self, sid, n):
        if sid not in self.live:
            return
        before = (self.pool.length(sid), self.pool.pages(sid), self.pool.num_free_pages)
        try:
            slots = self.pool.allocate(sid, n)
        except self.pc.OutOfPagesError:
            # exhaustion changes nothing
            assert (self.pool.length(sid), self.pool.pages(sid),
                    self.pool.num_free_pages) == before
            return
        start = before[0]
        pos = np.arange(start, start + n)
        pages = np.array(self.pool.pages(sid))
        assert np.array_equal(slots, pages[pos // BS] * BS + pos % BS)

    @rule(sid=consumes(seqs))
    def free(self, sid):
        if sid not in self.live:
            return
        self.pool.free(sid)
        self.live.discard(sid)

    @precondition(lambda self: len(self.live) < MAX_SEQS)
    @rule(target=seqs, src=seqs)
    def fork(self, src):
        if src not in self.live:
            return self._new_id()  # a dead id: later rules skip it
        dst = self._new_id()
        free_before = self.pool.num_free_pages
        try:
            self.pool.fork(src, dst)
        except self.pc.OutOfPagesError:
            assert not self.pool.has_sequence(dst) and self.pool.num_free_pages == free_before
            return dst
        self.live.add(dst)
        s_pages, d_pages = self.pool.pages(src), self.pool.pages(dst)
        full = self.pool.length(src) // BS
        assert d_pages[:full] == s_pages[:full]  # full pages shared
        assert self.pool.length(dst) == self.pool.length(src)
        if self.pool.length(src) % BS:
            assert d_pages[full] not in s_pages  # the partial page copied to a fresh page
        return dst

    @rule(sid=seqs, window=st.integers(1, 100), n_sink=st.integers(0, 20))
    def release(self, sid, window, n_sink):
        if sid not in self.live:
            return
        before = list(self.pool.pages(sid))
        self.pool.release_outside_window(sid, window, n_sink)
        after = self.pool.pages(sid)
        vis = orc.visible(self.pool.length(sid), window, n_sink)
        # a page goes exactly when none of its positions is visible; released pages stay gone
        for j, p in enumerate(before):
            seen = bool(vis[j * BS:(j + 1) * BS].any())
            assert after[j] == (p if (seen or p < 0) else -1), (j, p, after[j], window, n_sink)

    @rule()
    def compact(self):
        entries = {(s, j): p for s in self.live for j, p in enumerate(self.pool.pages(s))}
        src, dst = self.pool.compaction_moves()
        self.pool.compact()
        after = {(s, j): p for s in self.live for j, p in enumerate(self.pool.pages(s))}
        assert entries.keys() == after.keys()
        # one renaming f of page ids explains every entry: pages below n_used keep their
        # id, the k-th referenced page at or above n_used takes the k-th free id below it
        used = sorted({p for p in entries.values() if p >= 0})
        n_used = len(used)
        f = {p: p for p in used if p < n_used}
        f.update(zip(src, dst))
        assert sorted(f) == used and sorted(f.values()) == list(range(n_used))
        assert src == sorted(src) and dst == sorted(dst)
        for key, p in entries.items():
            assert after[key] == (f[p] if p >= 0 else -1), key
        assert sorted(self.pool._free) == list(range(n_used, NUM_PAGES))

    @invariant()
    def consistent(self):
        pool = self.pool
        ref = np.zeros(NUM_PAGES, dtype=np.int64)
        where = {}
        for s in self.live:
            pages = pool.pages(s)
            length = pool.length(s)
            assert len(pages) == -(-length // BS)
            bt, ctx = pool.tables([s])
            assert list(bt[0, :len(pages)]) == pages and (bt[0, len(pages):] == -1).all()
            assert ctx[0] == length
            for j, p in enumerate(pages):
                if p >= 0:
                    ref[p] += 1
                    where.setdefault(p, []).append((s, j))
        assert np.array_equal(ref, pool._ref)
        free = pool._free
        assert len(free) == len(set(free))
        assert set(free) == set(np.nonzero(ref == 0)[0].tolist())
        for p, owners in where.items():
            if len(owners) > 1:
                js = {j for _, j in owners}
                assert len(js) == 1  # shared at the same logical index
                j = js.pop()
                assert all(pool.length(s) >= (j + 1) * BS for s, _ in owners)  # a full page


TestPool = PoolMachine.TestCase
TestPool.settings = settings(max_examples=150, stateful_step_count=40, deadline=None,
                             suppress_health_check=[HealthCheck.too_slow])


# ------------------------------------------------------------------------------ oracle

@st.composite
def paged_case(draw, max_seqs=4, max_len=90):
    lengths = draw(st.lists(st.integers(0, max_len), min_size=1, max_size=max_seqs))
    hkv = draw(st.sampled_from([1, 2, 4]))
    d = draw(st.sampled_from([8, 16, 32]))
    bs = draw(st.sampled_from([4, 16]))
    dtype = draw(st.sampled_from([np.float32, np.float16]))
    extra = draw(st.integers(0, 4))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    rng = np.random.default_rng(seed)
    need = sum(-(-n // bs) for n in lengths)
    num_pages = need + extra + 1
    perm = rng.permutation(num_pages)
    mb = max(max(-(-n // bs) for n in lengths), 1)
    bt = np.full((len(lengths), mb), -1, dtype=np.int64)
    cur = 0
    for b, n in enumerate(lengths):
        k = -(-n // bs)
        bt[b, :k] = perm[cur:cur + k]
        cur += k
    n_tok = sum(lengths)
    k_new = rng.standard_normal((n_tok, hkv, d)).astype(dtype)
    v_new = rng.standard_normal((n_tok, hkv, d)).astype(dtype)
    slots = np.array([bt[b, p // bs] * bs + p % bs for b, n in enumerate(lengths) for p in range(n)],
                     dtype=np.int64)
    k_pool, v_pool = orc.empty_pools(num_pages, hkv, d, bs, dtype, fill=np.nan)
    orc.append(k_pool, v_pool, k_new, v_new, slots)
    return dict(lengths=lengths, hkv=hkv, d=d, bs=bs, dtype=dtype, bt=bt, ctx=np.array(lengths),
                k_new=k_new, v_new=v_new, k_pool=k_pool, v_pool=v_pool, rng=rng,
                num_pages=num_pages)


@settings(max_examples=40, deadline=None)
@given(paged_case())
def test_gather_of_append_returns_the_rows(c):
    k_out, v_out = orc.gather(c["k_pool"], c["v_pool"], c["bt"], c["ctx"], out_len=max(c["lengths"]))
    t = 0
    for b, n in enumerate(c["lengths"]):
        assert np.array_equal(k_out[b, :, :n].transpose(1, 0, 2).view(np.uint8),
                              c["k_new"][t:t + n].view(np.uint8))
        assert np.array_equal(v_out[b, :, :n].transpose(1, 0, 2).view(np.uint8),
                              c["v_new"][t:t + n].view(np.uint8))
        assert (k_out[b, :, n:] == 0).all() and (v_out[b, :, n:] == 0).all()
        t += n


def _relabel(c):
    """The same logical content under a random permutation of physical page ids."""
    pi = c["rng"].permutation(c["num_pages"])
    k2, v2 = np.empty_like(c["k_pool"]), np.empty_like(c["v_pool"])
    k2[pi] = c["k_pool"]
    v2[pi] = c["v_pool"]
    bt2 = np.where(c["bt"] >= 0, pi[np.maximum(c["bt"], 0)], -1)
    return k2, v2, bt2


def _q(c, g):
    return c["rng"].standard_normal((len(c["lengths"]), c["hkv"] * g, c["d"]))


@settings(max_examples=30, deadline=None)
@given(paged_case(), st.sampled_from([1, 2, 3]), st.integers(0, 40), st.integers(0, 6))
def test_page_relabelling_changes_nothing(c, g, window, n_sink):
    q = _q(c, g)
    k2, v2, bt2 = _relabel(c)
    n = max(c["lengths"])
    a = orc.gather(c["k_pool"], c["v_pool"], c["bt"], c["ctx"], out_len=n)
    b = orc.gather(k2, v2, bt2, c["ctx"], out_len=n)
    assert all(np.array_equal(x.view(np.uint8), y.view(np.uint8)) for x, y in zip(a, b))
    o1 = orc.decode_attention(q, c["k_pool"], c["v_pool"], c["bt"], c["ctx"], window=window,
                              n_sink=n_sink)
    o2 = orc.decode_attention(q, k2, v2, bt2, c["ctx"], window=window, n_sink=n_sink)
    assert np.array_equal(o1, o2)


@settings(max_examples=30, deadline=None)
@given(paged_case(), st.sampled_from([1, 4]))
def test_covering_windows_and_sinks_equal_no_window(c, g):
    q = _q(c, g)
    base = orc.decode_attention(q, c["k_pool"], c["v_pool"], c["bt"], c["ctx"])
    longest = max(c["lengths"])
    for window, n_sink in ((longest, 0), (longest + 7, 3), (1, longest)):
        out = orc.decode_attention(q, c["k_pool"], c["v_pool"], c["bt"], c["ctx"],
                                   window=window, n_sink=n_sink)
        assert np.array_equal(out, base), (window, n_sink)


@settings(max_examples=30, deadline=None)
@given(paged_case(), st.sampled_from([1, 2]), st.floats(-3.0, 3.0), st.floats(0.25, 4.0),
       st.integers(0, 30), st.integers(0, 4))
def test_linear_in_v_and_scale_moves_into_q(c, g, alpha, s, window, n_sink):
    assume(abs(alpha) > 1e-3)
    q = _q(c, g)
    kw = dict(window=window, n_sink=n_sink)
    sc = 1.0 / math.sqrt(c["d"])
    base = orc.decode_attention(q, c["k_pool"], c["v_pool"], c["bt"], c["ctx"], scale=sc, **kw)
    v_scaled = (c["v_pool"].astype(np.float64) * alpha)
    lin = orc.decode_attention(q, c["k_pool"], v_scaled, c["bt"], c["ctx"], scale=sc, **kw)
    assert np.allclose(lin, alpha * base, rtol=1e-9, atol=1e-12)
    moved = orc.decode_attention(q * s, c["k_pool"], c["v_pool"], c["bt"], c["ctx"], scale=sc / s, **kw)
    assert np.allclose(moved, base, rtol=1e-9, atol=1e-12)


@settings(max_examples=25, deadline=None)
@given(paged_case(max_seqs=3, max_len=60), st.sampled_from([1, 2]), st.integers(0, 30),
       st.integers(0, 4), st.data())
def test_prefill_rows_are_decodes_at_their_positions(c, g, window, n_sink, data):
    chunks = [data.draw(st.integers(0, n)) for n in c["lengths"]]
    qs = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int64)
    q = c["rng"].standard_normal((int(qs[-1]), c["hkv"] * g, c["d"]))
    out = orc.prefill_attention(q, c["k_pool"], c["v_pool"], c["bt"], c["ctx"], qs,
                                window=window, n_sink=n_sink)
    for b, (n, L) in enumerate(zip(chunks, c["lengths"])):
        for i in range(n):
            pos = L - n + i
            row = out[qs[b] + i]
            if pos < 0:
                assert (row == 0).all()
                continue
            dec = orc.decode_attention(q[qs[b] + i][None], c["k_pool"], c["v_pool"], c["bt"][b:b + 1],
                                       np.array([pos + 1]), window=window, n_sink=n_sink)
            assert np.allclose(row, dec[0], rtol=1e-12, atol=1e-12)
