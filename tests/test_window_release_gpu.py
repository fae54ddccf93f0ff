"""Sliding-window page release on the GPU: pages outside [0, n_sink) and the window go back
to the pool, and nothing a later query computes changes.

Semantics pinned (reference: the window / sink masks of src/core/attention.py:83-93,
115-148, sink_tokens = 4 as src/core/hrm_controller.py:172 produces): a decode query of
a sequence of length L sees [0, n_sink) and [L - window, L); a prefill row at position p
sees [0, n_sink) and [p - window + 1, p].  Positions only move forward, so the pages
wholly between the sink pages and L - window are never read again.

  * pool level, a C4-like table (bf16, GQA 32/8, head_dim 128, window 4096 + 4 sinks,
    contexts up to 20k): two pools with the same content, one released.  Decode
    attention, the fused append + attend step, and a later chunk's prefill (split and
    single-launch) give bit-identical outputs on the released pool, whose new pages come
    from the freed ones (LIFO reuse);
  * model level: hip_paged generation with a sliding window and sinks gives logits
    bit-identical to the same cache with release_window=False, while the released
    cache's resident pages stay at the window + sink pages;
  * a forward with a larger window than the released one is refused;
  * a released table stays valid through fork (the fork shares the resident pages and
    keeps the released entries) and compaction (the resident pages move down, the
    released entries stay -1): decode attention is bit-identical to the unreleased pool's;
  * the model-level check on FP8 pages too (scaling factors of released pages are never
    read again).
"""
from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

WINDOW, SINKS, BS = 4096, 4, 16
LENGTHS = [5000, 9000, 20000]
HQ, HKV, D = 32, 8, 128


@pytest.fixture(scope="module")
def PC(iva):
    from importlib import import_module
    return import_module("iva_amd.paged_cache")


def rows(n, seed, dev, dtype):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(n, HKV, D, generator=g, device=dev) * 0.5).to(dtype)


def filled_pool(PC, iva, dev, dtype, num_pages, max_seqs=len(LENGTHS)):
    pool = PC.PagedKVPool(num_pages, HKV, D, BS, 1, dtype, dev, max_seqs=max_seqs,
                          max_blocks_per_seq=math.ceil((max(LENGTHS) + 512) / BS))
    for i, n in enumerate(LENGTHS):
        pool.add_sequence(i)
        slots = torch.from_numpy(pool.allocate(i, n)).to(dev)
        iva.kv_append(rows(n, 100 + i, dev, dtype), rows(n, 200 + i, dev, dtype),
                      pool.k_pools[0], pool.v_pools[0], slots)
    return pool


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_release_keeps_decode_and_prefill_bit_identical(PC, iva, dev, dtype):
    need = sum(math.ceil((n + 300) / BS) for n in LENGTHS) + 8
    full = filled_pool(PC, iva, dev, dtype, need)
    rel = filled_pool(PC, iva, dev, dtype, need)
    ids = list(range(len(LENGTHS)))
    free0 = rel.num_free_pages
    before = {i: rel.pages(i) for i in ids}
    released = sum(rel.release_outside_window(i, WINDOW, SINKS) for i in ids)
    released_ids = {p for i in ids for p, q in zip(before[i], rel.pages(i)) if q < 0}
    assert len(released_ids) == released
    sink_pages = math.ceil(SINKS / BS)
    expect = sum(max(0, (n - WINDOW) // BS - sink_pages) for n in LENGTHS)
    assert released == expect > 0
    assert rel.num_free_pages == free0 + released
    bt_rel, ctx = rel.device_tables(ids)
    bt_full, ctx_full = full.device_tables(ids)
    assert torch.equal(ctx, ctx_full)
    for i, n in enumerate(LENGTHS):   # released entries are -1, the rest unchanged
        n_pages = math.ceil(n / BS)
        row_rel, row_full = bt_rel[i, :n_pages].cpu(), bt_full[i, :n_pages].cpu()
        gone = row_rel < 0
        assert int(gone.sum()) == max(0, (n - WINDOW) // BS - sink_pages)
        assert not bool(gone[:sink_pages].any()) and not bool((row_full < 0).any())
        assert torch.equal(row_rel[~gone], row_full[~gone])   # same allocation order

    g = torch.Generator(device=dev).manual_seed(7)
    q = (torch.randn(len(LENGTHS), HQ, D, generator=g, device=dev) * 0.5).to(dtype)
    kw = dict(window=WINDOW, n_sink=SINKS)
    o_full = iva.paged_decode_attention(q, full.k_pools[0], full.v_pools[0], bt_full, ctx, **kw)
    o_rel = iva.paged_decode_attention(q, rel.k_pools[0], rel.v_pools[0], bt_rel, ctx, **kw)
    assert torch.equal(o_full.view(torch.int16), o_rel.view(torch.int16))

    # a later chunk of 200 tokens: the released pool allocates from its freed pages
    chunk = 200
    for pool in (full, rel):
        for i in ids:
            slots = torch.from_numpy(pool.allocate(i, chunk)).to(dev)
            iva.kv_append(rows(chunk, 300 + i, dev, dtype), rows(chunk, 400 + i, dev, dtype),
                          pool.k_pools[0], pool.v_pools[0], slots)
    new_pages = {p for i in ids for p in rel.pages(i)[len(before[i]):]}
    assert new_pages and new_pages <= released_ids   # LIFO: the freed pages come back first
    assert rel.num_free_pages > full.num_free_pages
    bt_full, ctx = full.device_tables(ids)
    bt_rel, _ = rel.device_tables(ids)
    qs = torch.arange(0, (len(ids) + 1) * chunk, chunk, dtype=torch.int32, device=dev)
    qc = (torch.randn(len(ids) * chunk, HQ, D, generator=g, device=dev) * 0.5).to(dtype)
    for split in (True, False):
        a = iva.paged_prefill_attention(qc, full.k_pools[0], full.v_pools[0], bt_full, ctx, qs,
                                        max_query_len=chunk, split=split, **kw)
        b = iva.paged_prefill_attention(qc, rel.k_pools[0], rel.v_pools[0], bt_rel, ctx, qs,
                                        max_query_len=chunk, split=split, **kw)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"prefill split={split}"

    # the fused decode step (append at position L-1 + attend) on both pools
    for pool in (full, rel):
        for i in ids:
            pool.allocate(i, 1)
    bt_full, ctx = full.device_tables(ids)
    bt_rel, _ = rel.device_tables(ids)
    k_new, v_new = rows(len(ids), 500, dev, dtype), rows(len(ids), 600, dev, dtype)
    a = iva.paged_decode_append_attention(q, k_new, v_new, full.k_pools[0], full.v_pools[0],
                                          bt_full, ctx, **kw)
    b = iva.paged_decode_append_attention(q, k_new, v_new, rel.k_pools[0], rel.v_pools[0],
                                          bt_rel, ctx, **kw)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # the window and sink rows read back the same from both pools (released rows: zeros)
    kf, vf = iva.kv_gather(full.k_pools[0], full.v_pools[0], bt_full, ctx)
    kr, vr = iva.kv_gather(rel.k_pools[0], rel.v_pools[0], bt_rel, ctx)
    for i, n in enumerate(ctx.tolist()):
        # resident: the sink pages and every page from the one holding position
        # LENGTHS[i] - WINDOW (the window at the release) on
        keep = torch.zeros(kf.shape[2], dtype=torch.bool, device=dev)
        keep[:sink_pages * BS] = True
        keep[((LENGTHS[i] - WINDOW) // BS) * BS:n] = True
        assert torch.equal(kf[i][:, keep], kr[i][:, keep]) and torch.equal(vf[i][:, keep], vr[i][:, keep])
        assert not bool(kr[i][:, ~keep].any()), "released positions gather as zeros"


def test_release_then_fork_and_compact(PC, iva, dev):
    dtype = torch.bfloat16
    need = sum(math.ceil(n / BS) for n in LENGTHS) + 8
    full = filled_pool(PC, iva, dev, dtype, need)
    rel = filled_pool(PC, iva, dev, dtype, need, max_seqs=len(LENGTHS) + 1)
    ids = list(range(len(LENGTHS)))
    released = sum(rel.release_outside_window(i, WINDOW, SINKS) for i in ids)
    assert released > 0
    fork_of = 1                     # 9000 tokens: a partial last page, copied by the fork
    rel.fork(fork_of, len(LENGTHS))
    assert LENGTHS[fork_of] % BS and rel.pages(len(LENGTHS))[-1] != rel.pages(fork_of)[-1]
    assert rel.pages(len(LENGTHS))[:-1] == rel.pages(fork_of)[:-1]   # -1 entries included
    live = rel.num_pages - rel.num_free_pages
    moved = rel.compact()
    assert moved > 0 and rel.num_pages - rel.num_free_pages == live
    for i in ids + [len(LENGTHS)]:   # resident pages now below `live`, released ones -1
        pg = rel.pages(i)
        n = LENGTHS[i] if i < len(LENGTHS) else LENGTHS[fork_of]
        assert all(p < live for p in pg)
        assert sum(p < 0 for p in pg) == (n - WINDOW) // BS - math.ceil(SINKS / BS)

    g = torch.Generator(device=dev).manual_seed(11)
    q = (torch.randn(len(LENGTHS), HQ, D, generator=g, device=dev) * 0.5).to(dtype)
    kw = dict(window=WINDOW, n_sink=SINKS)
    # the same batch shape on both pools (the walk's split, and so its rounding, depends
    # on the batch): the unreleased pool lists the forked sequence's source twice
    q4 = torch.cat([q, q[fork_of:fork_of + 1]])
    bt_full, ctx = full.device_tables(ids + [fork_of])
    o_full = iva.paged_decode_attention(q4, full.k_pools[0], full.v_pools[0], bt_full, ctx, **kw)
    bt_rel, ctx_rel = rel.device_tables(ids + [len(LENGTHS)])
    assert torch.equal(ctx, ctx_rel)
    o_rel = iva.paged_decode_attention(q4, rel.k_pools[0], rel.v_pools[0], bt_rel, ctx_rel, **kw)
    assert torch.equal(o_full.view(torch.int16), o_rel.view(torch.int16))


@pytest.fixture(scope="module")
def M(iva):
    from importlib import import_module
    return import_module("iva_amd.model")


@pytest.mark.parametrize("pages", ["bf16", "fp8"])
def test_model_window_release(M, PC, dev, pages):
    cfg = dict(d_model=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, seq_len=1024,
               dropout=0.0, sliding_window=48, sink_tokens=4, attn_impl="hip_paged")
    if pages == "fp8":
        cfg["kv_cache_dtype"] = "fp8"
    page_dtype = torch.float8_e4m3fn if pages == "fp8" else torch.bfloat16
    torch.manual_seed(0)
    model = M.Transformer(M.TransformerConfig(**cfg)).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, 512, (3, 300), device=dev)

    def run(release):
        cache = PC.PagedKVCache(3, 2, 64, 0, dev, page_dtype, num_layers=2, max_seq_len=300,
                                release_window=release, compute_dtype=torch.bfloat16)
        resident = []
        with torch.no_grad():
            outs = [model(ids[:, :100], kv_cache=cache)["logits"]]
            resident.append(cache.resident_pages())
            for t in range(100, 300):
                outs.append(model(ids[:, t:t + 1], kv_cache=cache)["logits"])
                resident.append(cache.resident_pages())
        return torch.cat(outs, dim=1), cache, resident

    l_keep, c_keep, r_keep = run(False)
    l_rel, c_rel, r_rel = run(True)
    assert c_rel.pool.fp8 == (pages == "fp8")
    assert torch.equal(l_keep.view(torch.int16), l_rel.view(torch.int16))
    assert c_rel.seq_len == c_keep.seq_len == 300
    assert r_keep[-1] == 3 * math.ceil(300 / 16)
    # resident: the sink page plus the pages of the last 48 positions (and the partly
    # visible one below them), per sequence
    assert max(r_rel[1:]) <= 3 * (1 + math.ceil(48 / 16) + 1)
    assert c_rel.pool.num_free_pages > c_keep.pool.num_free_pages
    with pytest.raises(ValueError, match="released"):
        c_rel.note_window(96, 4)
    with pytest.raises(ValueError, match="released"):
        c_rel.note_window(None, 0)
    c_rel.note_window(32, 4)   # a smaller window sees a subset: allowed
    c_keep.free()
    c_rel.free()


def test_graph_decode_releases_at_the_end(M, dev):
    cfg = dict(d_model=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, seq_len=1024,
               dropout=0.0, sliding_window=32, sink_tokens=4, attn_impl="hip_paged")
    torch.manual_seed(1)
    model = M.Transformer(M.TransformerConfig(**cfg)).to(dev, torch.bfloat16).eval()
    prompts = torch.randint(0, 512, (2, 64), device=dev)
    with torch.no_grad():
        a = model.generate(prompts, max_length=96, do_sample=False, eos_token_id=None,
                           use_graph=True)
        b = model.generate(prompts, max_length=96, do_sample=False, eos_token_id=None)
    assert torch.equal(a, b)
