"""Pins the CPU oracle (no GPU).  Each check is independent of the formula it pins:
brute-force loops over the documented address formula, round trips, the
reference's own contiguous KVCache restatement, a library routine (torch SDPA),
closed forms, invariances, and golden fixtures.  Planted mistakes in the oracle
must make at least one check fail."""
from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_kv as orc
from oracle import reference_path as rp

GOLDEN = Path(__file__).resolve().parent / "golden"


def rand_case(seed, lengths, hkv, d, bs, dtype=np.float32, extra=3):
    rng = np.random.default_rng(seed)
    need = sum(-(-n // bs) for n in lengths)
    num_pages = need + extra
    perm = rng.permutation(num_pages)
    mb = max(-(-n // bs) for n in lengths) if lengths else 1
    bt = np.full((len(lengths), max(mb, 1)), -1, dtype=np.int64)
    cur = 0
    for b, n in enumerate(lengths):
        k = -(-n // bs)
        bt[b, :k] = perm[cur:cur + k]
        cur += k
    n_tok = sum(lengths)
    k_new = rng.standard_normal((n_tok, hkv, d)).astype(dtype)
    v_new = rng.standard_normal((n_tok, hkv, d)).astype(dtype)
    slots = np.concatenate([[bt[b, p // bs] * bs + p % bs for p in range(n)]
                            for b, n in enumerate(lengths)]).astype(np.int64) if n_tok else np.zeros(0, np.int64)
    return dict(bt=bt, ctx=np.array(lengths, dtype=np.int64), k_new=k_new, v_new=v_new, slots=slots,
                num_pages=num_pages)


# ------------------------------------------------------------------ append / gather

@pytest.mark.parametrize("dtype,d,bs", [(np.float32, 8, 4), (np.float16, 16, 16), (np.float32, 12, 3)])
def test_append_gather_vs_address_formula_loops(dtype, d, bs):
    c = rand_case(1, [5, 1, 9], 2, d, bs, dtype)
    slots = c["slots"].copy()
    slots[2] = -1
    kp, vp = orc.empty_pools(c["num_pages"], 2, d, bs, dtype, fill=7)
    orc.append(kp, vp, c["k_new"], c["v_new"], slots)
    kf, vf = orc.empty_pools(c["num_pages"], 2, d, bs, dtype, fill=7)
    kf, vf = kf.reshape(-1), vf.reshape(-1)
    orc.append_loops(kf, vf, c["k_new"], c["v_new"], slots, c["num_pages"], 2, d, bs)
    assert np.array_equal(kp.reshape(-1), kf) and np.array_equal(vp.reshape(-1), vf)
    bt = c["bt"].copy()
    bt[2, 0] = -4  # invalid page
    ko, vo = orc.gather(kp, vp, bt, c["ctx"], out_len=12)
    lk, lv = orc.gather_loops(kf, vf, bt, c["ctx"], c["num_pages"], 2, d, bs, 12)
    assert np.array_equal(ko, lk) and np.array_equal(vo, lv)


def test_round_trip_and_canary():
    c = rand_case(2, [17, 64, 129, 200], 8, 64, 16)
    kp, vp = orc.empty_pools(c["num_pages"], 8, 64, 16, np.float32, fill=np.float32(-3.5))
    orc.append(kp, vp, c["k_new"], c["v_new"], c["slots"])
    ko, vo = orc.gather(kp, vp, c["bt"], c["ctx"])
    start = 0
    for b, n in enumerate(c["ctx"]):
        assert np.array_equal(ko[b, :, :n], c["k_new"][start:start + n].transpose(1, 0, 2))
        assert np.array_equal(vo[b, :, :n], c["v_new"][start:start + n].transpose(1, 0, 2))
        assert not ko[b, :, n:].any()
        start += n
    # pages no sequence owns keep the canary in every word
    used = set(c["bt"][c["bt"] >= 0].tolist())
    for p in range(c["num_pages"]):
        if p not in used:
            assert (kp[p] == -3.5).all() and (vp[p] == -3.5).all()


def test_page_permutation_invariance():
    """The same logical content under two different page assignments gathers identically."""
    a = rand_case(3, [40, 7], 2, 16, 8)
    b = dict(a)
    rng = np.random.default_rng(99)
    perm = rng.permutation(a["num_pages"])
    b_bt = np.where(a["bt"] >= 0, perm[np.maximum(a["bt"], 0)], -1)
    b_slots = perm[a["slots"] // 8] * 8 + a["slots"] % 8
    outs = []
    for bt, slots in ((a["bt"], a["slots"]), (b_bt, b_slots)):
        kp, vp = orc.empty_pools(a["num_pages"], 2, 16, 8, np.float32)
        orc.append(kp, vp, a["k_new"], a["v_new"], slots)
        outs.append(orc.gather(kp, vp, bt, a["ctx"]))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_gather_matches_reference_kvcache():
    """Paged gather == the reference's contiguous KVCache (rope_kv.py:98-137) fed with the
    same rows through update() in uneven chunks (exercising its grow-by-copy resize)."""
    c = rand_case(4, [17, 64, 129, 200], 8, 64, 16)
    kp, vp = orc.empty_pools(c["num_pages"], 8, 64, 16, np.float32)
    orc.append(kp, vp, c["k_new"], c["v_new"], c["slots"])
    ko, vo = orc.gather(kp, vp, c["bt"], c["ctx"])
    start = 0
    for b, n in enumerate(c["ctx"].tolist()):
        cache = rp.ContiguousKVCache(1, 8, 64, 0, dtype=torch.float32)
        rows_k = torch.from_numpy(c["k_new"][start:start + n]).permute(1, 0, 2).unsqueeze(0)
        rows_v = torch.from_numpy(c["v_new"][start:start + n]).permute(1, 0, 2).unsqueeze(0)
        pos = 0
        for chunk in (1, 3, 16, 50, 1000):
            e = min(n, pos + chunk)
            if e > pos:
                cache.update(rows_k[:, :, pos:e], rows_v[:, :, pos:e], pos)
            pos = e
        ck, cv = cache.get_slice(0, n)
        assert np.array_equal(ck[0].numpy(), ko[b, :, :n]) and np.array_equal(cv[0].numpy(), vo[b, :, :n])
        start += n


def test_c1_golden_digests():
    """The oracle reproduces the committed C1 digests from the seed."""
    import __graft_entry__
    iva = __graft_entry__.load_package()
    gold = json.loads((GOLDEN / "c1.json").read_text())
    w = iva.workloads.c1_append_gather(seed=gold["seed"])
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    k_new, v_new = w["k_new"].numpy().view(np.uint32), w["v_new"].numpy().view(np.uint32)
    assert sha(k_new) == gold["k_new_sha256"] and sha(v_new) == gold["v_new_sha256"]
    assert w["layout"].block_tables.tolist() == gold["block_tables"]
    kp, vp = orc.empty_pools(64, 8, 64, 16, np.uint32)
    orc.append(kp, vp, k_new, v_new, w["slot_mapping"].numpy())
    ko, vo = orc.gather(kp, vp, w["layout"].block_tables.numpy(), w["layout"].context_lens.numpy())
    assert sha(ko) == gold["k_out_sha256"] and sha(vo) == gold["v_out_sha256"]


# ------------------------------------------------------------------ decode attention

def attn_case(seed, lengths, hq, hkv, d, bs=16, scale_vals=1.0):
    c = rand_case(seed, lengths, hkv, d, bs)
    c["k_new"] *= scale_vals
    kp, vp = orc.empty_pools(c["num_pages"], hkv, d, bs, np.float32)
    orc.append(kp, vp, c["k_new"], c["v_new"], c["slots"])
    rng = np.random.default_rng(seed + 1000)
    c.update(kp=kp, vp=vp, q=rng.standard_normal((len(lengths), hq, d)), hq=hq, hkv=hkv, d=d)
    return c


def sdpa_reference(c, scale=None, window=0, n_sink=0):
    """torch.nn.functional.scaled_dot_product_attention in fp64 on the gathered rows."""
    ko, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
    out = np.zeros((len(c["ctx"]), c["hq"], c["d"]))
    g = c["hq"] // c["hkv"]
    for b, n in enumerate(c["ctx"].tolist()):
        if n == 0:
            continue
        k = torch.from_numpy(ko[b, :, :n]).double().repeat_interleave(g, 0)
        v = torch.from_numpy(vo[b, :, :n]).double().repeat_interleave(g, 0)
        q = torch.from_numpy(c["q"][b]).double().unsqueeze(1)
        j = torch.arange(n)
        mask = (j >= n - window) | (j < n_sink) if window else torch.ones(n, dtype=torch.bool)
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.view(1, 1, n), scale=scale)
        out[b] = o.squeeze(1).numpy()
    return out


def check_sdpa(fn, seed=5):
    ok = True
    for lengths, hq, hkv, d, window, sink in (([1, 20, 77], 8, 2, 16, 0, 0),
                                              ([90, 33, 5], 4, 4, 8, 10, 3),
                                              ([64, 200], 6, 2, 32, 31, 0)):
        c = attn_case(seed, lengths, hq, hkv, d)
        got = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"], window=window, n_sink=sink)
        ok &= np.allclose(got, sdpa_reference(c, window=window, n_sink=sink), atol=1e-10)
    return ok


def check_closed_forms(fn):
    ok = True
    # one key -> v[0]
    c = attn_case(6, [1], 4, 2, 8)
    got = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"])
    _, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
    ok &= np.allclose(got[0], np.repeat(vo[0, :, 0], 2, axis=0), atol=1e-12)
    # identical keys -> mean of v (per kv head)
    c = attn_case(7, [37], 4, 2, 8)
    c["kp"][:] = c["kp"][c["bt"][0, 0], :, :, :1, :][None]
    got = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"])
    _, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
    ok &= np.allclose(got[0], np.repeat(vo[0, :, :37].mean(axis=1), 2, axis=0), atol=1e-12)
    # one dominant score -> that row's v: key 13 of kv head h is 60*q of query head 2h
    c = attn_case(8, [40], 4, 2, 8)
    ko, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
    rows_k = ko[0].transpose(1, 0, 2).copy()  # [L, Hkv, D]
    for h in range(2):
        rows_k[13, h] = 60.0 * c["q"][0, 2 * h]
    kp, vp = orc.empty_pools(c["num_pages"], 2, 8, 16, np.float32)
    slots = np.array([c["bt"][0, p // 16] * 16 + p % 16 for p in range(40)])
    orc.append(kp, vp, rows_k.astype(np.float32), vo[0].transpose(1, 0, 2), slots)
    got = fn(c["q"], kp, vp, c["bt"], c["ctx"])
    for h in range(2):
        ok &= np.allclose(got[0, 2 * h], vo[0, h, 13], atol=1e-6)
    return ok


def check_window_brute_force(fn):
    """Window/sink sets vs pure-Python term-by-term evaluation on tiny inputs."""
    ok = True
    for window, sink in ((3, 0), (4, 2), (1, 1), (50, 1)):
        c = attn_case(9 + window, [11, 3, 20], 4, 2, 4, bs=4)
        ko, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
        exp = orc.decode_attention_loops(c["q"].tolist(), ko.tolist(), vo.tolist(), c["ctx"].tolist(),
                                         1 / math.sqrt(4), window, sink)
        got = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"], window=window, n_sink=sink)
        ok &= np.allclose(got, np.array(exp), atol=1e-12)
    return ok


def check_reference_path(fn):
    """Agreement with the restated reference path (torch.cat append + AttentionTorch math)."""
    lengths = [30, 7, 64]
    c = attn_case(11, lengths, 8, 2, 16)
    ko, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
    lmax = max(lengths)
    cache_k = torch.zeros(3, 2, lmax - 1, 16, dtype=torch.float64)
    cache_v = torch.zeros_like(cache_k)
    valid = torch.zeros(3, lmax - 1, dtype=torch.bool)
    k_new = torch.zeros(3, 2, 1, 16, dtype=torch.float64)
    v_new = torch.zeros_like(k_new)
    for b, n in enumerate(lengths):
        cache_k[b, :, :n - 1] = torch.from_numpy(ko[b, :, :n - 1])
        cache_v[b, :, :n - 1] = torch.from_numpy(vo[b, :, :n - 1])
        valid[b, :n - 1] = True
        k_new[b, :, 0] = torch.from_numpy(ko[b, :, n - 1])
        v_new[b, :, 0] = torch.from_numpy(vo[b, :, n - 1])
    ok = True
    for window, sink in ((None, 0), (9, 2)):
        ref = rp.reference_decode_step(cache_k, cache_v, valid, torch.tensor(lengths),
                                       torch.from_numpy(c["q"]).unsqueeze(2), k_new, v_new,
                                       1 / math.sqrt(16), window=window, n_sink=sink)
        got = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"], window=window or 0, n_sink=sink)
        ok &= np.allclose(got, ref.squeeze(2).numpy(), atol=1e-12)
    return ok


def check_permutation(fn):
    c = attn_case(12, [70, 19], 4, 2, 8)
    got_a = fn(c["q"], c["kp"], c["vp"], c["bt"], c["ctx"])
    perm = np.random.default_rng(5).permutation(c["num_pages"])
    inv = np.argsort(perm)
    kp2, vp2 = c["kp"][inv], c["vp"][inv]  # page p moves to index perm[p]
    bt2 = np.where(c["bt"] >= 0, perm[np.maximum(c["bt"], 0)], -1)
    got_b = fn(c["q"], kp2, vp2, bt2, c["ctx"])
    return np.allclose(got_a, got_b, atol=1e-13)


PIN_CHECKS = [check_sdpa, check_closed_forms, check_window_brute_force, check_reference_path,
              check_permutation]


@pytest.mark.parametrize("check", PIN_CHECKS, ids=lambda f: f.__name__)
def test_decode_oracle_pins(check):
    assert check(orc.decode_attention)


def test_decode_golden_fixture():
    g = np.load(GOLDEN / "decode_tiny.npz")
    got = orc.decode_attention(g["q"], g["k_pool"], g["v_pool"], g["block_tables"],
                               g["context_lens"], window=int(g["window"]), n_sink=int(g["n_sink"]))
    assert np.allclose(got, g["expected"], atol=1e-12)


def _mutant_no_scale(q, kp, vp, bt, ctx, scale=None, window=0, n_sink=0):
    return orc.decode_attention(q, kp, vp, bt, ctx, scale=1.0, window=window, n_sink=n_sink)


def _mutant_swap_kv(q, kp, vp, bt, ctx, scale=None, window=0, n_sink=0):
    # K pages read as if they were V pages and vice versa (transposed operand roles)
    p, h, nch, bs, x = kp.shape
    kp2 = vp.reshape(p, h, nch, x, bs).transpose(0, 1, 2, 4, 3).copy()
    vp2 = kp.transpose(0, 1, 2, 4, 3).reshape(p, h, nch * x, bs).copy()
    return orc.decode_attention(q, kp2, vp2, bt, ctx, scale=scale, window=window, n_sink=n_sink)


@pytest.mark.parametrize("mutant", ["no_scale", "gqa_tile", "window_off_by_one", "sink_and",
                                    "swap_kv"])
def test_planted_mistakes_are_caught(monkeypatch, mutant):
    fn = orc.decode_attention
    if mutant == "no_scale":
        fn = _mutant_no_scale
    elif mutant == "swap_kv":
        fn = _mutant_swap_kv
    elif mutant == "gqa_tile":
        monkeypatch.setattr(orc, "expand_gqa", lambda x, g: np.concatenate([x] * g, axis=0))
    elif mutant == "window_off_by_one":
        real = orc.visible
        monkeypatch.setattr(orc, "visible",
                            lambda n, w=0, s=0: real(n, w - 1, s) if w and w > 1 else real(n, w, s))
    elif mutant == "sink_and":
        # the reference's successive masked_fill ANDs the sink mask into the window mask,
        # which drops the sinks (attention.py:83-93)
        real = orc.visible
        monkeypatch.setattr(orc, "visible", lambda n, w=0, s=0: real(n, w, 0))
    results = [check(fn) for check in PIN_CHECKS]
    assert not all(results), f"planted mistake {mutant} passed every pin check"


# ------------------------------------------------------------------ index ops

def test_index_ops_vs_torch():
    rng = np.random.default_rng(13)
    kv = rng.standard_normal((2, 3, 10, 8)).astype(np.float32)
    idx = np.array([9, 0, 4, 4, 7])
    got = orc.index_gather(kv, idx)
    assert np.array_equal(got, torch.from_numpy(kv)[:, :, torch.from_numpy(idx)].numpy())
    for j, i in enumerate(idx):
        assert np.array_equal(got[:, :, j], kv[:, :, i])
    uniq = np.array([9, 0, 4, 7])
    vals = rng.standard_normal((2, 3, 4, 8)).astype(np.float32)
    out = orc.index_scatter(kv, uniq, vals)
    ref = torch.from_numpy(kv).clone()
    ref[:, :, torch.from_numpy(uniq)] = torch.from_numpy(vals)
    assert np.array_equal(out, ref.numpy())
    assert not np.shares_memory(out, kv)


# ------------------------------------------------------------------ prefill attention

def prefill_case(seed, lengths, chunks, hq, hkv, d, bs=16):
    """Pools holding `lengths` tokens per sequence; query rows for the last chunks[b]
    positions of each sequence (chunks[b] may exceed the length: negative positions)."""
    c = attn_case(seed, lengths, hq, hkv, d, bs)
    rng = np.random.default_rng(seed + 2000)
    qs = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int64)
    c.update(qp=rng.standard_normal((int(qs[-1]), hq, d)), qs=qs, chunks=list(chunks))
    return c


def _call_pf(fn, c, **kw):
    return fn(c["qp"], c["kp"], c["vp"], c["bt"], c["ctx"], c["qs"], **kw)


def check_pf_rows_are_decodes(fn):
    """Row i of sequence b at position p equals the (separately pinned) decode oracle
    with context length p + 1 on the same pages; negative positions give zero rows."""
    ok = True
    for lengths, chunks, hq, hkv, d, window, sink in (
            ([20, 37, 5], [20, 9, 1], 4, 2, 8, 0, 0),
            ([50, 33], [17, 33], 6, 2, 8, 7, 3),
            ([3, 40], [5, 0], 2, 2, 4, 0, 0),
            ([64], [64], 4, 1, 8, 16, 1)):
        c = prefill_case(31, lengths, chunks, hq, hkv, d)
        c["bt"][-1, 1] = -1 if c["bt"].shape[1] > 1 else c["bt"][-1, 1]  # an invalid page
        got = _call_pf(fn, c, window=window, n_sink=sink)
        for b, (length, n) in enumerate(zip(lengths, chunks)):
            for i in range(n):
                row = int(c["qs"][b]) + i
                pos = length - n + i
                if pos < 0:
                    ok &= not got[row].any()
                    continue
                exp = orc.decode_attention(c["qp"][row][None], c["kp"], c["vp"], c["bt"][b:b + 1],
                                           np.array([pos + 1]), window=window, n_sink=sink)
                ok &= np.allclose(got[row], exp[0], atol=1e-12)
    return ok


def check_pf_sdpa_causal(fn):
    """Full prefill (chunk = whole sequence) vs torch SDPA in fp64: is_causal for plain
    causal attention; otherwise an explicit mask, the reference's window loop
    (attention.py:120-127) united with the first n_sink positions."""
    ok = True
    for length, hq, hkv, d, window, sink in ((45, 4, 2, 8, 0, 0), (60, 6, 3, 8, 9, 2),
                                             (33, 2, 1, 16, 1, 1)):
        c = prefill_case(37, [length], [length], hq, hkv, d)
        got = _call_pf(fn, c, window=window, n_sink=sink)
        ko, vo = orc.gather(c["kp"], c["vp"], c["bt"], c["ctx"])
        g = hq // hkv
        k = torch.from_numpy(ko[0, :, :length]).double().repeat_interleave(g, 0)
        v = torch.from_numpy(vo[0, :, :length]).double().repeat_interleave(g, 0)
        q = torch.from_numpy(c["qp"]).double().transpose(0, 1)  # [Hq, L, D]
        if not window:
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        else:
            mask = torch.zeros(length, length, dtype=torch.bool)
            for i in range(length):                          # attention.py:120-127
                mask[i, max(0, i - window + 1):i + 1] = True
                mask[i, :min(sink, i + 1)] = True            # sinks, never past i
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        ok &= np.allclose(got, o.transpose(0, 1).numpy(), atol=1e-10)
    return ok


def check_pf_chunking(fn):
    """A sequence prefilled in two chunks gives the rows of one full prefill."""
    c = prefill_case(41, [70], [70], 4, 2, 8)
    full = _call_pf(fn, c, window=20, n_sink=2)
    c1 = dict(c, ctx=np.array([33]), qs=np.array([0, 33]), qp=c["qp"][:33])
    c2 = dict(c, ctx=np.array([70]), qs=np.array([0, 37]), qp=c["qp"][33:])
    parts = np.concatenate([_call_pf(fn, c1, window=20, n_sink=2),
                            _call_pf(fn, c2, window=20, n_sink=2)])
    return np.allclose(full, parts, atol=1e-12)


PF_CHECKS = [check_pf_rows_are_decodes, check_pf_sdpa_causal, check_pf_chunking]


@pytest.mark.parametrize("check", PF_CHECKS, ids=lambda f: f.__name__)
def test_prefill_oracle_pins(check):
    assert check(orc.prefill_attention)


def _pf_mutant_relative(q, kp, vp, bt, ctx, qs, scale=None, window=0, n_sink=0):
    # the reference's literal torch.tril over [S, S_cache + S] (attention.py:79-81):
    # chunk row i sees keys 0..i, ignoring the cached prefix
    ctx = np.asarray(ctx)
    out = np.zeros(q.shape)
    for b in range(len(ctx)):
        for i in range(int(qs[b + 1] - qs[b])):
            out[qs[b] + i] = orc.decode_attention(q[qs[b] + i][None], kp, vp, bt[b:b + 1],
                                                  np.array([i + 1]), scale, window, n_sink)[0]
    return out


@pytest.mark.parametrize("mutant", ["relative_positions", "window_off_by_one", "sinks_dropped",
                                    "gqa_tile", "causal_inclusive_off"])
def test_prefill_planted_mistakes_are_caught(monkeypatch, mutant):
    fn = orc.prefill_attention
    real = orc.visible_at
    if mutant == "relative_positions":
        fn = _pf_mutant_relative
    elif mutant == "window_off_by_one":
        monkeypatch.setattr(orc, "visible_at",
                            lambda p, n, w=0, s=0: real(p, n, w + 1 if w else w, s))
    elif mutant == "sinks_dropped":
        monkeypatch.setattr(orc, "visible_at", lambda p, n, w=0, s=0: real(p, n, w, 0))
    elif mutant == "gqa_tile":
        monkeypatch.setattr(orc, "expand_gqa", lambda x, g: np.concatenate([x] * g, axis=0))
    elif mutant == "causal_inclusive_off":
        monkeypatch.setattr(orc, "visible_at", lambda p, n, w=0, s=0: real(p - 1, n, w, s))
    results = [check(fn) for check in PF_CHECKS]
    assert not all(results), f"planted mistake {mutant} passed every prefill pin check"


# ------------------------------------------------------------------ FP8 pools

def test_e4m3_decode_matches_torch_exhaustively():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = orc.e4m3_decode(codes)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.array_equal(ref[~np.isnan(ref)], got[~np.isnan(got)])


def test_e4m3_encode_matches_torch_rounding():
    """Every representable value, every midpoint (ties to even) and its neighbours,
    subnormals and random values in [-448, 448] round as torch's float8_e4m3fn cast."""
    vals = np.unique(orc.e4m3_decode(np.arange(256, dtype=np.uint8)))
    vals = vals[~np.isnan(vals)]
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(0)
    xs = np.concatenate([vals, mids, np.nextafter(mids, np.float32(np.inf)),
                         np.nextafter(mids, np.float32(-np.inf)),
                         rng.uniform(-448, 448, 50000).astype(np.float32),
                         (rng.standard_normal(20000) * 0.01).astype(np.float32),
                         np.array([2.0 ** -10, 2.0 ** -12, 1e-30, 0.0, -0.0], np.float32)])
    xs = xs[np.abs(xs) <= 448]
    ref = torch.from_numpy(xs).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.e4m3_encode(xs), ref)
    # beyond +-448 this build saturates (torch's cast gives NaN from 464 on)
    assert orc.e4m3_encode(np.array([470.0, -1e9, np.inf], np.float32)).tolist() == [0x7E, 0xFE, 0x7E]


def test_row_scale_is_the_reference_rule():
    """fp8_runtime.py:66-76: sf = 448 / amax, 1 for amax == 0, clamped to [1e-8, 1e8]
    by max(1e-8, min(sf, 1e8)) -- evaluated here with Python's own min / max on every
    amax, non-finite ones included (a NaN sf comes out as 1e-8)."""
    amax = np.array([0.0, 1.0, 448.0, 3.5, 1e-12, 1e12, np.inf, np.nan], np.float32)

    def reference(a):  # the rule's own steps, in Python floats
        if a == 0:
            return 1.0
        sf = 448.0 / a if a != np.inf else 0.0
        return max(1e-8, min(sf, 1e8))
    exp = np.array([reference(float(a)) for a in amax], np.float32)
    exp[3] = np.float32(448.0) / np.float32(3.5)  # the build divides in float32
    assert np.array_equal(orc.row_scale(amax), exp)


def test_fp8_rows_round_trip_and_layout():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((40, 2, 32)) * np.array([1e-3, 50.0])[None, :, None]).astype(np.float32)
    x[3] = 0.0
    codes, sf = orc.quantize_rows(x)
    back = orc.e4m3_decode(codes) / sf[..., None]
    amax = np.abs(x).max(axis=-1, keepdims=True)
    assert np.all(np.abs(back - x) <= 2.0 ** -4 * np.abs(x) + 2.0 ** -9 / 448 * amax + 1e-30)
    assert np.all(codes[3] == 0) and np.all(sf[3] == 1)
    # append_fp8 = quantize + the (pinned) append address formula + factors at [page, head, row]
    c = rand_case(4, [7, 20], 2, 32, 16)
    kp, vp = orc.empty_pools(c["num_pages"], 2, 32, 16, np.uint8)
    ks, vs = orc.empty_scales(c["num_pages"], 2, 16), orc.empty_scales(c["num_pages"], 2, 16)
    orc.append_fp8(kp, vp, ks, vs, c["k_new"], c["v_new"], c["slots"])
    kc, ksf = orc.quantize_rows(c["k_new"])
    kf, vf = orc.empty_pools(c["num_pages"], 2, 32, 16, np.uint8)
    kf, vf = kf.reshape(-1), vf.reshape(-1)
    vc, vsf = orc.quantize_rows(c["v_new"])
    orc.append_loops(kf, vf, kc, vc, c["slots"], c["num_pages"], 2, 32, 16)
    assert np.array_equal(kp.reshape(-1), kf)
    assert np.array_equal(orc.fp8_v_from_tiles(vp).reshape(-1), vf)   # V in the FP8 tile order
    for t, s in enumerate(c["slots"]):
        assert np.array_equal(ks[s // 16, :, s % 16], ksf[t]) and np.array_equal(vs[s // 16, :, s % 16], vsf[t])


def test_fp8_v_tile_order_gives_each_lane_consecutive_words():
    """The FP8 V tile order is a permutation of the tile's bytes (round trip exact) in
    which lane (ln, lq) of the decode walk finds its operand words -- keys 4lq..4lq+3 of
    dims ln, 16 + ln, ..., one word per 16 dims -- as consecutive bytes, lanes in order."""
    for d in (64, 128, 256):
        nat = np.arange(d * 16, dtype=np.int32).reshape(1, 1, d, 16)
        dev = orc.fp8_v_to_tiles(nat)
        assert np.array_equal(orc.fp8_v_from_tiles(dev), nat)
        flat = dev.reshape(-1)
        assert np.array_equal(np.sort(flat), np.arange(d * 16))
        nb = d // 16
        for ln in range(16):
            for lq in range(4):
                words = flat[(ln * 4 + lq) * nb * 4:(ln * 4 + lq + 1) * nb * 4].reshape(nb, 4)
                want = nat[0, 0, 16 * np.arange(nb)[:, None] + ln, 4 * lq + np.arange(4)[None, :]]
                assert np.array_equal(words, want)


# ------------------------------------------------------------------ RoPE

def test_rope_matches_the_reference_module():
    """oracle.rope vs the reference's RoPE module restated in torch float32
    (reference_path.ReferenceRoPE = rope_kv.py:9-50), at positions up to 70k."""
    rng = np.random.default_rng(21)
    for d, theta in ((64, 10000.0), (128, 500000.0), (16, 10.0)):
        x = rng.standard_normal((2, 3, 40, d)).astype(np.float32)
        pos = np.stack([np.arange(40), rng.integers(0, 70000, 40)]).astype(np.int64)
        ref = rp.ReferenceRoPE(d, theta).forward(torch.from_numpy(x), torch.from_numpy(pos)).numpy()
        for b in range(2):
            got = orc.rope(x[b].transpose(1, 0, 2), pos[b], theta).transpose(1, 0, 2)
            assert np.allclose(got, ref[b], rtol=0, atol=2e-6 * max(1.0, np.abs(x).max()))


def _rope_check_d2_rotates_by_p(fn):
    """D 2, any theta: the one pair has frequency theta^0 = 1, so position p rotates it by
    p radians counter-clockwise: (1, 0) -> (cos p, sin p), (0, 1) -> (-sin p, cos p)."""
    p = np.array([1, 2, 7, 100], dtype=np.int64)
    e0 = fn(np.tile([[1.0, 0.0]], (4, 1)), p, 10000.0)
    e1 = fn(np.tile([[0.0, 1.0]], (4, 1)), p, 10000.0)
    a = p.astype(np.float64)
    return (np.allclose(e0, np.stack([np.cos(a), np.sin(a)], 1), atol=1e-6)
            and np.allclose(e1, np.stack([-np.sin(a), np.cos(a)], 1), atol=1e-6))


def _rope_check_pair_frequencies(fn):
    """D 4 / 8 at theta 10000: pair j turns at theta^(-2j/D), so at D 4 pair 1 turns by
    0.01 p, and at D 8 pairs 1, 2, 3 by 0.1 p, 0.01 p, 0.001 p; a unit vector on the even
    dim of pair j lands on (cos a_j, sin a_j) and leaves the other pairs at zero."""
    ok = True
    for d, rates in ((4, [1.0, 0.01]), (8, [1.0, 0.1, 0.01, 0.001])):
        for j, rate in enumerate(rates):
            x = np.zeros((3, d))
            x[:, 2 * j] = 1.0
            p = np.array([0, 100, 1000], dtype=np.int64)
            y = fn(x, p, 10000.0)
            a = p * rate
            want = np.zeros((3, d))
            want[:, 2 * j], want[:, 2 * j + 1] = np.cos(a), np.sin(a)
            ok = ok and np.allclose(y, want, atol=1e-4)
    return ok


def _rope_check_composition(fn):
    """R(p) then R(q) is R(p + q) (a rotation group), and R(p) is orthogonal: checked on
    random rows at D 16 where the float32 angles are exact (p * f_i with small p)."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal((5, 16))
    p, q = np.array([1, 2, 3, 4, 5]), np.array([3, 1, 4, 1, 5])
    two = fn(fn(x, p, 10.0), q, 10.0)
    one = fn(x, p + q, 10.0)
    return np.allclose(two, one, atol=1e-5) and np.allclose(
        np.linalg.norm(fn(x, p, 10.0), axis=1), np.linalg.norm(x, axis=1))


ROPE_PINS = [_rope_check_d2_rotates_by_p, _rope_check_pair_frequencies, _rope_check_composition]


@pytest.mark.parametrize("check", ROPE_PINS, ids=lambda f: f.__name__)
def test_rope_oracle_pins(check):
    assert check(orc.rope)


def _rope_mutant(kind):
    """Plausible mistakes in a RoPE restatement, each of which a pin must catch."""
    def fn(x, positions, theta=10000.0):
        x = np.asarray(x, dtype=np.float64)
        d = x.shape[-1]
        j = np.arange(d // 2)
        expo = (j / d) if kind == "exponent_i_over_d" else (2 * j / d)
        f = (1.0 / theta ** expo).astype(np.float32)
        ang = np.asarray(positions, np.float64)[:, None] * f[None, :]
        c, s = np.cos(ang), np.sin(ang)
        if kind == "rotate_half":   # pairs (i, i + D/2) instead of (2i, 2i + 1)
            x0, x1 = x[..., :d // 2], x[..., d // 2:]
        else:
            x0, x1 = x[..., 0::2], x[..., 1::2]
        sg = -1.0 if kind == "sign_flip" else 1.0
        y0, y1 = x0 * c - sg * x1 * s, sg * x0 * s + x1 * c
        y = np.empty_like(x)
        if kind == "rotate_half":
            y[..., :d // 2], y[..., d // 2:] = y0, y1
        else:
            y[..., 0::2], y[..., 1::2] = y0, y1
        return y
    return fn


@pytest.mark.parametrize("kind", ["sign_flip", "exponent_i_over_d", "rotate_half"])
def test_rope_planted_mistakes_are_caught(kind):
    fn = _rope_mutant(kind)
    assert not all(check(fn) for check in ROPE_PINS), f"planted RoPE mistake {kind} passed"
    assert all(check(_rope_mutant("none")) for check in ROPE_PINS)   # the harness itself


def test_rope_invariants():
    rng = np.random.default_rng(22)
    x = rng.standard_normal((10, 4, 32))
    assert np.allclose(orc.rope(x, np.zeros(10, np.int64)), x, atol=0)     # position 0
    y = orc.rope(x, rng.integers(0, 5000, 10))
    assert np.allclose(np.hypot(y[..., 0::2], y[..., 1::2]), np.hypot(x[..., 0::2], x[..., 1::2]))
    # relative position: <R(p) q, R(p') k> depends only on p - p' (up to the float32
    # rounding of the angles, ~1e-5 rad at these positions)
    q, k = rng.standard_normal(32), rng.standard_normal(32)
    a = (orc.rope(q[None, None], [100])[0, 0] * orc.rope(k[None, None], [37])[0, 0]).sum()
    b = (orc.rope(q[None, None], [163])[0, 0] * orc.rope(k[None, None], [100])[0, 0]).sum()
    c = (orc.rope(q[None, None], [163])[0, 0] * orc.rope(k[None, None], [37])[0, 0]).sum()
    assert abs(a - b) < 1e-4 and abs(a - c) > 1e-2
