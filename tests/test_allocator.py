"""PagedKVPool bookkeeping on the CPU (no device storage): LIFO free list, block
tables and slot ids, reference-counted fork, window release, exhaustion errors,
config sizing and state round trip.  Slot ids are checked against the address
rule slot = page * block_size + position % block_size."""
from __future__ import annotations

import numpy as np
import pytest


def pool(iva, pages=16, **kw):
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    kw.setdefault("max_seqs", 8)
    return pc.PagedKVPool(pages, 2, 64, 16, allocate_storage=False, device="cpu", **kw), pc


def test_allocate_slots_follow_pages(iva):
    p, _ = pool(iva)
    p.add_sequence("a")
    s = p.allocate("a", 20)                     # 2 pages
    pages = p.pages("a")
    assert len(pages) == 2 and p.length("a") == 20
    pos = np.arange(20)
    assert np.array_equal(s, np.array(pages)[pos // 16] * 16 + pos % 16)
    s2 = p.allocate("a", 13)                    # 33 tokens -> 3 pages
    assert len(p.pages("a")) == 3 and s2[0] == pages[1] * 16 + 4
    bt, ctx = p.tables(["a"])
    assert list(bt[0, :3]) == p.pages("a") and ctx[0] == 33


def test_lifo_free_list_reuses_last_freed(iva):
    p, _ = pool(iva)
    for name in "abc":
        p.add_sequence(name)
        p.allocate(name, 16)
    freed = p.pages("b")
    p.free("b")
    p.add_sequence("d")
    p.allocate("d", 1)
    assert p.pages("d") == freed                # most recently freed page first
    assert p.num_free_pages == 16 - 3


def test_exhaustion_is_atomic(iva):
    p, pc = pool(iva, pages=4)
    p.add_sequence("a")
    p.allocate("a", 48)                         # 3 pages
    p.add_sequence("b")
    with pytest.raises(pc.OutOfPagesError):
        p.allocate("b", 40)                     # needs 3, 1 free
    assert p.length("b") == 0 and p.pages("b") == [] and p.num_free_pages == 1


def test_negative_counts_are_refused_and_zero_is_a_no_op(iva):
    p, _ = pool(iva)
    p.add_sequence("a")
    p.allocate("a", 5)
    before = (p.length("a"), p.pages("a"), p.num_free_pages)
    with pytest.raises(ValueError, match="n_tokens"):
        p.allocate("a", -1)
    with pytest.raises(ValueError, match="n_tokens"):
        p.reserve("a", -3)
    assert (p.length("a"), p.pages("a"), p.num_free_pages) == before
    assert len(p.allocate("a", 0)) == 0
    assert (p.length("a"), p.pages("a"), p.num_free_pages) == before


def test_block_table_width_limit(iva):
    p, pc = pool(iva, max_blocks_per_seq=2)
    p.add_sequence("a")
    p.allocate("a", 32)
    with pytest.raises(pc.OutOfPagesError, match="block table"):
        p.allocate("a", 1)


def test_fork_shares_full_pages_and_copies_partial(iva):
    p, _ = pool(iva)
    p.add_sequence("a")
    p.allocate("a", 40)                         # pages 0,1 full, page 2 partial
    pa = p.pages("a")
    p.fork("a", "b")
    pb = p.pages("b")
    assert pb[:2] == pa[:2] and pb[2] != pa[2] and p.length("b") == 40
    p.free("a")                                 # shared pages stay with b
    assert set(pb[:2]).isdisjoint(p._free)
    assert pa[2] in p._free
    p.free("b")
    assert p.num_free_pages == 16


def test_release_outside_window_keeps_sinks_and_window(iva):
    p, _ = pool(iva, pages=32)
    p.add_sequence("a")
    p.allocate("a", 300)                        # pages 0..18
    released = p.release_outside_window("a", window=64, n_sink=4)
    # visible: [0, 4) on page 0 and [236, 300) on pages 14..18
    assert released == 14 - 1
    pages = p.pages("a")
    assert pages[0] >= 0 and all(x < 0 for x in pages[1:14]) and all(x >= 0 for x in pages[14:])
    bt, _ = p.tables(["a"])
    assert (bt[0, 1:14] == -1).all()
    with pytest.raises(IndexError):
        p.slots("a", [100])                     # released page
    assert p.release_outside_window("a", window=64, n_sink=4) == 0


def test_rows_and_state_round_trip(iva):
    p, _ = pool(iva)
    p.add_sequence(("x", 1))
    p.allocate(("x", 1), 17)
    p.add_sequence("y")
    p.allocate("y", 5)
    st = p.state_dict()
    q, _ = pool(iva)
    q.load_state_dict(st)
    assert q.pages(("x", 1)) == p.pages(("x", 1)) and q.length("y") == 5
    assert np.array_equal(q.tables(["y", ("x", 1)])[0], p.tables(["y", ("x", 1)])[0])
    with pytest.raises(ValueError):
        pool(iva, pages=8)[0].load_state_dict(st)


def test_from_config_honours_quant_infer_memory_block(iva):
    """configs/quant_infer.yaml:50-54: paged_kv_cache, kv_cache_dtype, kv_cache_size,
    kv_cache_blocks."""
    from importlib import import_module
    import torch
    pc = import_module("iva_amd.paged_cache")
    cfg = {"paged_kv_cache": True, "kv_cache_dtype": "bf16", "kv_cache_size": 1024,
           "kv_cache_blocks": 256}
    p = pc.PagedKVPool.from_config(cfg, num_layers=2, num_kv_heads=8, head_dim=128, device="cpu")
    assert p.num_pages == 256 and p.max_blocks == 64 and p.dtype == torch.bfloat16
    assert len(p.k_pools) == 2 and p.k_pools[0].shape == (256, 8, 16, 16, 8)
    # kv_cache_dtype "fp8" (the file's own value): e4m3fn pages + per-(slot, head) factors
    p8 = pc.PagedKVPool.from_config(dict(cfg, kv_cache_dtype="fp8"), 1, 8, 128, device="cpu")
    assert p8.fp8 and p8.k_pools[0].dtype == torch.float8_e4m3fn
    assert p8.k_pools[0].shape == (256, 8, 8, 16, 16) and p8.v_pools[0].shape == (256, 8, 128, 16)
    assert p8.k_scales[0].shape == (256, 8, 16) and p8.k_scales[0].dtype == torch.float32
    with pytest.raises(NotImplementedError, match="fp4"):
        pc.PagedKVPool.from_config(dict(cfg, kv_cache_dtype="fp4"), 1, 8, 128, device="cpu")
    with pytest.raises(ValueError):
        pc.PagedKVPool.from_config(dict(cfg, paged_kv_cache=False), 1, 8, 128, device="cpu")


def test_churn_keeps_tables_consistent(iva):
    """Random adds / appends / frees: every live page is owned exactly once, the free
    list and the owned pages partition the pool, tables mirror the page lists."""
    rng = np.random.default_rng(0)
    p, pc = pool(iva, pages=64, max_seqs=16)
    live = {}
    for step in range(400):
        op = rng.integers(3)
        if op == 0 and len(live) < 16:
            sid = ("s", step)
            p.add_sequence(sid)
            live[sid] = 0
        elif op == 1 and live:
            sid = list(live)[rng.integers(len(live))]
            n = int(rng.integers(1, 40))
            try:
                p.allocate(sid, n)
                live[sid] += n
            except pc.OutOfPagesError:
                pass
        elif live:
            sid = list(live)[rng.integers(len(live))]
            p.free(sid)
            del live[sid]
        owned = [x for s in live for x in p.pages(s)]
        assert len(owned) == len(set(owned))
        assert sorted(owned + p._free) == list(range(64))
        for s, n in live.items():
            assert p.length(s) == n
            bt, ctx = p.tables([s])
            assert list(bt[0, :len(p.pages(s))]) == p.pages(s) and ctx[0] == n


def test_compaction_moves_pack_live_pages(iva):
    """After churn, compaction moves every live page above n_used to a free id below it
    (disjoint sets); the renumbered tables keep each sequence's page order, and the
    free list becomes the tail [n_used, P)."""
    rng = np.random.default_rng(7)
    p, pc = pool(iva, pages=64, max_seqs=64)
    live = []
    for step in range(60):
        if p.num_free_pages < 8:
            break
        sid = ("s", step)
        p.add_sequence(sid)
        p.allocate(sid, int(rng.integers(1, 60)))
        live.append(sid)
        if len(live) > 3:
            p.free(live.pop(int(rng.integers(len(live)))))
    p.fork(live[0], "fork")                      # shared pages (refcount 2) move once
    before = {s: p.pages(s) for s in live + ["fork"]}
    src, dst = p.compaction_moves()
    n_used = int((p._ref > 0).sum())
    assert set(src).isdisjoint(dst) and len(src) == len(dst)
    assert all(s >= n_used for s in src) and all(d < n_used for d in dst)
    moved = p.compact()
    assert moved == len(src)
    remap = dict(zip(src, dst))
    for s, pages in before.items():
        assert p.pages(s) == [remap.get(x, x) for x in pages]
        bt, _ = p.tables([s])
        assert list(bt[0, :len(pages)]) == p.pages(s)
    owned = {x for s in before for x in p.pages(s)}
    assert owned == set(range(n_used))
    assert sorted(p._free) == list(range(n_used, 64))
    p.add_sequence("new")
    p.allocate("new", 1)
    assert p.pages("new") == [n_used]             # allocation continues from the tail
    assert p.compact() == 0


def test_generation_moves_with_every_table_change(iva):
    """Every block-table change bumps the pool generation (device copies of the tables
    are keyed on it); a length-only change inside allocated pages does not."""
    p, _ = pool(iva, pages=32, max_seqs=8)
    g = [p.generation]

    def bumped():
        g.append(p.generation)
        return g[-1] > g[-2]

    p.add_sequence("a")
    assert bumped()
    p.allocate("a", 20)                          # new pages
    assert bumped()
    p.allocate("a", 3)                           # fits in the pages it has
    assert not bumped()
    p.add_sequence("b")
    p.allocate("b", 40)
    p.fork("a", "c")
    assert bumped()
    p.free("b")                                  # frees the low pages: a gap below "c"
    assert bumped()
    assert p.compact() > 0                       # renumbers "a" / "c" with no length change
    assert bumped()
    p.add_sequence("d")
    p.allocate("d", 16 * 6)
    assert p.release_outside_window("d", window=20, n_sink=0) > 0
    assert bumped()
    p.load_state_dict(p.state_dict())
    assert bumped()


def test_churn_driver_reaches_steady_state(iva):
    """The C5 driver's host bookkeeping (no device storage): sequences start at random
    points of their lifetimes, so from the first step on prefill chunks (<= 512 tokens,
    never past the prompt), decode tokens and completions all occur; lengths never pass
    their targets; completed sequences' pages return and are reused (fragmented tables)."""
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    wl = import_module("iva_amd.workloads")
    pool = pc.PagedKVPool(64000, 8, 128, 16, 1, allocate_storage=False, device="cpu",
                          max_seqs=512, max_blocks_per_seq=1024)
    churn = wl.ChurnBatch(pool, n_seqs=256, seed=0, fill=False)
    steps, done, n_pre, n_dec = 40, [], [], []
    for _ in range(steps):
        plan = churn.plan_step()
        assert all(0 < n <= 512 for _, n in plan["prefill"])
        assert len(plan["prefill_slots"]) == sum(n for _, n in plan["prefill"])
        assert len(plan["prefill"]) + len(plan["decode"]) == 256
        for sid, _ in plan["prefill"]:
            assert pool.length(sid) <= churn.prompt[sid]
        for sid in churn.ids:
            assert pool.length(sid) <= churn.target[sid]
        n_pre.append(len(plan["prefill"]))
        n_dec.append(len(plan["decode"]))
        done.append(churn.finish_step())
    assert min(n_pre) > 0 and min(n_dec) > 0
    assert sum(done) >= steps               # about two completions per step
    assert sum(1 for d in done if d > 0) >= steps * 0.7
    assert 1600 < churn.lognormal_mean() < 1700   # E[LogNormal(ln 1024, 1)] = 1688, capped
    for ids in (churn.ids[:64], churn.ids[-64:]):   # the oldest and the newest sequences
        bt, _ = pool.tables(ids)
        assert (np.diff(bt[:, :4], axis=1) != 1).mean() > 0.3


def test_cache_update_exhaustion_changes_nothing(iva):
    """PagedKVCache.update on a pool that cannot hold the whole batch's growth raises
    before any sequence grows (the check precedes every allocation and the append)."""
    import torch
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    cache = pc.PagedKVCache(3, 2, 16, 0, "cpu", torch.float32, num_layers=1, max_seq_len=64,
                            num_pages=5)
    before = [(cache.pool.length(s), cache.pool.pages(s)) for s in cache.seq_ids]
    free = cache.pool.num_free_pages
    rows = torch.zeros(3, 2, 32, 16)  # 32 tokens: 2 pages per sequence, 6 > 5
    with pytest.raises(pc.OutOfPagesError, match="batch needs 6 pages"):
        cache.update(rows, rows, 0)
    assert [(cache.pool.length(s), cache.pool.pages(s)) for s in cache.seq_ids] == before
    assert cache.pool.num_free_pages == free


def test_cache_window_policy_releases_and_guards(iva):
    """PagedKVCache's window release (host bookkeeping only): the noted window's
    invisible pages go back to the pool, the sink page stays, and a later forward may not
    widen the window or its sinks past what stayed resident."""
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    p = pc.PagedKVPool(64, 2, 64, 16, allocate_storage=False, device="cpu", max_seqs=8)
    cache = pc.PagedKVCache(2, 2, 64, 0, "cpu", pool=p)
    for s in cache.seq_ids:
        p.allocate(s, 300)                      # 19 pages each
    cache.seq_len = 300
    assert cache.resident_pages() == 38
    assert cache.release_window() == 0          # no window noted: nothing happens
    cache.note_window(64, 4)
    assert cache.window_policy == (64, 4)
    released = cache.release_window()
    # visible: [0, 4) and [236, 300) -> pages 0 and 14..18 stay
    assert released == 2 * 13 and cache.resident_pages() == 2 * 6
    assert all(p.pages(s)[1:14] == [-1] * 13 for s in cache.seq_ids)
    for bad in ((128, 4), (None, 0), (64, 17)):
        with pytest.raises(ValueError, match="released"):
            cache.note_window(*bad)
    cache.note_window(32, 16)                   # sinks within the kept page, smaller window
    keep = pc.PagedKVCache(1, 2, 64, 0, "cpu", pool=p, release_window=False)
    p.allocate(keep.seq_ids[0], 300)
    keep.seq_len = 300
    keep.note_window(64, 4)
    assert keep.release_window() == 0 and keep.resident_pages() == 19
    keep.note_window(None)                      # nothing was released: any window is fine
    c2 = pc.create_kv_cache(2, 2, 64, 0, "cpu", pool=p)
    assert isinstance(c2, pc.PagedKVCache) and c2.seq_len == 0 and c2.batch_size == 2
