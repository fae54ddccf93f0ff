"""Pools past 4 GiB: every paged op addresses pages whose offsets exceed 2^31 elements and
2^32 bytes (the sizes a 288 GB device holds in production).

Each op runs on the same logical content twice: in a pool pair of ≈4.4 GB per pool whose
sequences' pages sit at ids around and above the page whose bytes start at 2^32 (2^31
elements for 16-bit pages; plus a few low ids), and in a compact pool pair holding the same pages under other ids.  The kernels
visit the same logical pages in the same order either way, so every output must be
bit-identical between the two; the compact run is checked against the oracle as well.
Covered: append (plain and with RoPE), gather, decode attention (stream walk,
partitioned walk, window + sinks), the fused append + attend step, prefill (single
launch and split), page copies, and FP8 pages (append, gather, decode, prefill).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

LENGTHS = [300, 1000, 77]  # none a multiple of 16: the fused step's slot fits the last page
HKV, G, D, BS = 8, 4, 128, 16
FP8 = torch.float8_e4m3fn


def _ids(n_pages: int, page_bytes: int, seed: int):
    """Page ids for the large pool (most straddle or pass the page whose bytes start at
    2^32, a few are low) and for the compact pool (a permutation of 0 .. n - 1)."""
    gen = torch.Generator().manual_seed(seed)
    edge = (1 << 32) // page_bytes
    high = edge - 40 + torch.randperm(4000, generator=gen)[: n_pages - 8]
    low = torch.randperm(1000, generator=gen)[:8]
    large = torch.cat([high, low])[torch.randperm(n_pages, generator=gen)]
    small = torch.randperm(n_pages, generator=gen)
    return large.to(torch.int32), small.to(torch.int32), int(edge + 4000)


def _tables(ids: torch.Tensor):
    need = [-(-n // BS) for n in LENGTHS]
    bt = torch.full((len(LENGTHS), max(need)), -1, dtype=torch.int32)
    cur = 0
    for b, k in enumerate(need):
        bt[b, :k] = ids[cur:cur + k]
        cur += k
    return bt


def _slots(bt: torch.Tensor, lengths):
    return torch.cat([bt[b, torch.arange(n) // BS].long() * BS + torch.arange(n) % BS
                      for b, n in enumerate(lengths)]).to(torch.int32)


class Pools:
    """A large and a compact pool pair with the same appended content."""

    def __init__(self, iva, dev, dtype, seed=0):
        self.dtype = dtype
        fp8 = dtype == FP8
        page_elems = HKV * D * BS
        n_pages = sum(-(-n // BS) for n in LENGTHS)
        esize = 1 if fp8 else 2
        ids_l, ids_s, num_large = _ids(n_pages, page_elems * esize, seed)
        assert int(ids_l.max()) * page_elems * esize > (1 << 32)
        assert int(ids_l.max()) * page_elems > (1 << 31) or fp8
        self.bt_l, self.bt_s = _tables(ids_l).to(dev), _tables(ids_s).to(dev)
        self.ctx = torch.tensor(LENGTHS, dtype=torch.int32, device=dev)
        self.pools = {}
        for name, num in (("l", num_large), ("s", n_pages)):
            ks, vs = iva.pool_shapes(num, HKV, D, BS, dtype)
            k = torch.empty(ks, dtype=torch.uint8 if fp8 else dtype, device=dev)
            v = torch.empty(vs, dtype=torch.uint8 if fp8 else dtype, device=dev)
            used = (ids_l if name == "l" else ids_s).long().to(dev)
            k[used] = 0
            v[used] = 0
            if fp8:
                k, v = k.view(FP8), v.view(FP8)
                sc = [torch.ones(iva.scale_shape(num, HKV), device=dev) for _ in range(2)]
            else:
                sc = [None, None]
            self.pools[name] = (k, v, sc[0], sc[1])
        gen = torch.Generator().manual_seed(seed + 1)
        n_tok = sum(LENGTHS)
        src = torch.float16 if fp8 else dtype
        self.k_new = (torch.randn(n_tok, HKV, D, generator=gen) * D ** -0.5).to(src).to(dev)
        self.v_new = (torch.randn(n_tok, HKV, D, generator=gen) * D ** -0.5).to(src).to(dev)
        for name, bt in (("l", self.bt_l), ("s", self.bt_s)):
            k, v, ksc, vsc = self.pools[name]
            iva.kv_append(self.k_new, self.v_new, k, v, _slots(bt.cpu(), LENGTHS).to(dev),
                          k_scale=ksc, v_scale=vsc)

    def bt(self, name):
        return self.bt_l if name == "l" else self.bt_s

    def scales(self, name):
        k, v, ksc, vsc = self.pools[name]
        return {} if ksc is None else {"k_scale": ksc, "v_scale": vsc}


def same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bit-identical (NaN payloads included)."""
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.uint8),
                                              b.contiguous().view(torch.uint8))


@pytest.fixture(scope="module")
def p16(iva, dev):
    p = Pools(iva, dev, torch.float16, seed=3)
    yield p
    del p
    torch.cuda.empty_cache()


def test_append_and_gather(iva, dev, p16):
    outs = {}
    for name in ("l", "s"):
        k, v, _, _ = p16.pools[name]
        outs[name] = iva.kv_gather(k, v, p16.bt(name), p16.ctx, out_len=max(LENGTHS))
    assert same(outs["l"][0], outs["s"][0]) and same(outs["l"][1], outs["s"][1])
    t = 0
    for b, n in enumerate(LENGTHS):
        assert same(outs["l"][0][b, :, :n].transpose(0, 1), p16.k_new[t:t + n])
        assert same(outs["l"][1][b, :, :n].transpose(0, 1), p16.v_new[t:t + n])
        t += n


@pytest.mark.parametrize("kw", [{}, {"partition_pages": 8}, {"window": 200, "n_sink": 4}],
                         ids=["stream", "partitioned", "window"])
def test_decode(iva, dev, p16, kw):
    q = (torch.randn(len(LENGTHS), HKV * G, D, generator=torch.Generator().manual_seed(5))
         .to(torch.float16).to(dev))
    outs = {name: iva.paged_decode_attention(q, p16.pools[name][0], p16.pools[name][1],
                                             p16.bt(name), p16.ctx, **kw) for name in ("l", "s")}
    assert same(outs["l"], outs["s"])
    k, v, _, _ = p16.pools["s"]
    ref = orc.decode_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                               v.float().cpu().numpy(), p16.bt_s.cpu().numpy(),
                               p16.ctx.cpu().numpy(), window=kw.get("window", 0),
                               n_sink=kw.get("n_sink", 0))
    assert np.abs(outs["s"].float().cpu().numpy() - ref).max() <= 2e-3


def test_fused_step_and_prefill(iva, dev, p16):
    gen = torch.Generator().manual_seed(6)
    q = (torch.randn(len(LENGTHS), HKV * G, D, generator=gen) * 0.5).to(torch.float16).to(dev)
    k1 = (torch.randn(len(LENGTHS), HKV, D, generator=gen) * D ** -0.5).to(torch.float16).to(dev)
    v1 = (torch.randn(len(LENGTHS), HKV, D, generator=gen) * D ** -0.5).to(torch.float16).to(dev)
    ctx1 = p16.ctx + 1
    outs, rows = {}, {}
    for name in ("l", "s"):
        k, v, _, _ = p16.pools[name]
        outs[name] = iva.paged_decode_append_attention(q, k1, v1, k, v, p16.bt(name), ctx1)
        ko, vo = iva.kv_gather(k, v, p16.bt(name), ctx1, out_len=max(LENGTHS) + 1)
        rows[name] = (ko, vo)
    assert same(outs["l"], outs["s"])
    assert same(rows["l"][0], rows["s"][0]) and same(rows["l"][1], rows["s"][1])
    for b, n in enumerate(LENGTHS):
        assert same(rows["l"][0][b, :, n], k1[b]) and same(rows["l"][1][b, :, n], v1[b])
    # prefill: the last 64 positions of each sequence (through the fused step's token)
    chunk = 64
    qs = torch.arange(len(LENGTHS) + 1, dtype=torch.int32, device=dev) * chunk
    qp = (torch.randn(chunk * len(LENGTHS), HKV * G, D, generator=gen) * 0.5).to(torch.float16).to(dev)
    for split in (False, True):
        o = {name: iva.paged_prefill_attention(qp, p16.pools[name][0], p16.pools[name][1],
                                               p16.bt(name), ctx1, qs, split=split)
             for name in ("l", "s")}
        assert same(o["l"], o["s"]), f"split={split}"
    k, v, _, _ = p16.pools["s"]
    ref = orc.prefill_attention(qp.float().cpu().numpy(), k.float().cpu().numpy(),
                                v.float().cpu().numpy(), p16.bt_s.cpu().numpy(),
                                ctx1.cpu().numpy(), qs.cpu().numpy())
    assert np.abs(o["s"].float().cpu().numpy() - ref).max() <= 2e-3


def test_rope_append_and_page_copy(iva, dev, p16):
    """RoPE append of new rows into a fresh high page, then a copy of that page to
    another high id: the pages of the large pool equal the compact pool's."""
    gen = torch.Generator().manual_seed(8)
    kn = (torch.randn(BS, HKV, D, generator=gen)).to(torch.float16).to(dev)
    vn = (torch.randn(BS, HKV, D, generator=gen)).to(torch.float16).to(dev)
    pos = torch.arange(100, 100 + BS, dtype=torch.int32, device=dev)
    kl, vl, _, _ = p16.pools["l"]
    ks, vs, _, _ = p16.pools["s"]
    top = kl.shape[0] - 1
    used_l = set(p16.bt_l[p16.bt_l >= 0].tolist())
    src_l, dst_l = top, top - 1
    assert src_l not in used_l and dst_l not in used_l
    # the compact pool has no free page: borrow its page 0's content afterwards
    save_k, save_v = ks[0].clone(), vs[0].clone()
    iva.kv_append(kn, vn, kl, vl, (torch.arange(BS, device=dev) + src_l * BS).to(torch.int32),
                  rope_positions=pos)
    iva.kv_append(kn, vn, ks, vs, torch.arange(BS, dtype=torch.int32, device=dev),
                  rope_positions=pos)
    assert same(kl[src_l], ks[0]) and same(vl[src_l], vs[0])
    iva.copy_pages(kl, vl, torch.tensor([src_l], dtype=torch.int32, device=dev),
                   torch.tensor([dst_l], dtype=torch.int32, device=dev))
    assert same(kl[dst_l], ks[0]) and same(vl[dst_l], vs[0])
    ks[0].copy_(save_k)
    vs[0].copy_(save_v)


def test_fp8_pages(iva, dev):
    p = Pools(iva, dev, FP8, seed=11)
    try:
        outs = {}
        for name in ("l", "s"):
            k, v, _, _ = p.pools[name]
            outs[name] = iva.kv_gather(k, v, p.bt(name), p.ctx, out_len=max(LENGTHS),
                                       **p.scales(name))
        assert same(outs["l"][0], outs["s"][0]) and same(outs["l"][1], outs["s"][1])
        # codes and factors of the used pages: identical bytes
        for j in range(p.bt_s.shape[1]):
            for b in range(len(LENGTHS)):
                il, is_ = int(p.bt_l[b, j]), int(p.bt_s[b, j])
                if il < 0:
                    continue
                assert same(p.pools["l"][0][il], p.pools["s"][0][is_])
                assert same(p.pools["l"][1][il], p.pools["s"][1][is_])
                assert same(p.pools["l"][2][il], p.pools["s"][2][is_])
        q = (torch.randn(len(LENGTHS), HKV * G, D, generator=torch.Generator().manual_seed(12))
             .to(torch.float16).to(dev))
        dec = {name: iva.paged_decode_attention(q, p.pools[name][0], p.pools[name][1], p.bt(name),
                                                p.ctx, **p.scales(name)) for name in ("l", "s")}
        assert same(dec["l"], dec["s"])
        k, v, ksc, vsc = p.pools["s"]
        ref = orc.decode_attention_fp8(q.float().cpu().numpy(), k.view(torch.uint8).cpu().numpy(),
                                       v.view(torch.uint8).cpu().numpy(), ksc.cpu().numpy(),
                                       vsc.cpu().numpy(), p.bt_s.cpu().numpy(), p.ctx.cpu().numpy())
        assert np.abs(dec["s"].float().cpu().numpy() - ref).max() <= 2e-3
        qs = torch.arange(len(LENGTHS) + 1, dtype=torch.int32, device=dev) * 48
        qp = (torch.randn(48 * len(LENGTHS), HKV * G, D, generator=torch.Generator().manual_seed(13))
              * 0.5).to(torch.float16).to(dev)
        for split in (False, True):
            o = {name: iva.paged_prefill_attention(qp, p.pools[name][0], p.pools[name][1],
                                                   p.bt(name), p.ctx, qs, split=split,
                                                   **p.scales(name)) for name in ("l", "s")}
            assert same(o["l"], o["s"]), f"split={split}"
    finally:
        del p
        torch.cuda.empty_cache()


def test_index_gather_scatter_past_2g_elements(iva, dev):
    """kv_ops on a contiguous [B, H, S, D] cache of more than 2^31 elements: rows at the
    cache's far end gather and scatter exactly, and a scatter leaves every other byte
    of its copy as it was."""
    b, h, s, d = 2, 8, (1 << 20) + 64, 128
    assert b * h * s * d > (1 << 31)
    kv = torch.empty((b, h, s, d), dtype=torch.float16, device=dev)
    idx = torch.tensor([s - 1, 0, s - 17, 12345, s // 2], dtype=torch.int64, device=dev)
    gen = torch.Generator().manual_seed(21)
    rows = torch.randn(b, h, idx.numel(), d, generator=gen).to(torch.float16).to(dev)
    kv[:, :, idx] = rows
    assert same(iva.kv_ops(kv, idx), rows)
    vals = torch.randn(b, h, idx.numel(), d, generator=gen).to(torch.float16).to(dev)
    out = iva.kv_ops(kv, idx, vals, operation="scatter")
    assert same(out[:, :, idx], vals)
    out[:, :, idx] = rows
    assert same(out, kv)
    del kv, out
    torch.cuda.empty_cache()


def _torch_rows(k_pool, v_pool, bt_row, length):
    """[Hkv, L, D] fp32 K and V of one sequence by plain torch indexing of the pools."""
    n = -(-length // BS)
    pages = bt_row[:n].long()
    hkv, d = k_pool.shape[1], k_pool.shape[2] * k_pool.shape[4]
    k = k_pool[pages].permute(1, 0, 3, 2, 4).reshape(hkv, n * BS, d)[:, :length].float()
    v = v_pool[pages].permute(1, 0, 3, 2).reshape(hkv, n * BS, d)[:, :length].float()
    return k, v


def _torch_attention(q, k, v, positions):
    """fp32 causal attention of query rows q [R, Hq, D] at absolute positions over k, v
    [Hkv, L, D] (all keys <= the row's position)."""
    hq, hkv = q.shape[1], k.shape[0]
    kk = k.repeat_interleave(hq // hkv, dim=0)  # [Hq, L, D]
    vv = v.repeat_interleave(hq // hkv, dim=0)
    s = torch.matmul(q.float().permute(1, 0, 2).contiguous(), kk.transpose(1, 2).contiguous())
    s = s * q.shape[2] ** -0.5  # [Hq, R, L]
    j = torch.arange(k.shape[1], device=q.device)
    s = s.masked_fill(j[None, None, :] > positions[None, :, None], float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vv).permute(1, 0, 2)  # [R, Hq, D]


def test_million_token_context(iva, dev):
    """One sequence of 2^20 positions (65,536 pages in one table row) beside a short one:
    decode (stream and partitioned walks) and a 16-token chunk through the split prefill
    against fp32 torch attention on the GPU, and decode with a window + sinks against the
    fp64 oracle."""
    lengths = [1 << 20, 33]
    hkv, g, d = 2, 2, 64
    dd = iva.workloads.decode_batch(lengths, hkv * g, hkv, d, torch.float16, seed=31,
                                    device=dev, scale=d ** -0.5)
    lay = dd["layout"]
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    refs = []
    for b, n in enumerate(lengths):
        k, v = _torch_rows(dd["k_pool"], dd["v_pool"], bt[b], n)
        refs.append(_torch_attention(dd["q"][b:b + 1], k, v,
                                     torch.tensor([n - 1], device=dev))[0])
    ref = torch.stack(refs)
    for kw in ({}, {"partition_pages": 256}):
        out = iva.paged_decode_attention(dd["q"], dd["k_pool"], dd["v_pool"], bt, ctx, **kw)
        err = float((out.float() - ref).abs().max())
        assert err <= 2e-3, (kw, err)
    out = iva.paged_decode_attention(dd["q"], dd["k_pool"], dd["v_pool"], bt, ctx, window=70000,
                                     n_sink=5)
    oref = orc.decode_attention(dd["q"].float().cpu().numpy(), dd["k_pool"].float().cpu().numpy(),
                                dd["v_pool"].float().cpu().numpy(), lay.block_tables.numpy(),
                                lay.context_lens.numpy(), window=70000, n_sink=5)
    assert np.abs(out.float().cpu().numpy() - oref).max() <= 2e-3
    qs = torch.tensor([0, 16, 32], dtype=torch.int32, device=dev)
    qp = (torch.randn(32, hkv * g, d, generator=torch.Generator().manual_seed(32)) * 0.5)
    qp = qp.half().to(dev)
    out = iva.paged_prefill_attention(qp, dd["k_pool"], dd["v_pool"], bt, ctx, qs, split=True)
    for b, n in enumerate(lengths):
        k, v = _torch_rows(dd["k_pool"], dd["v_pool"], bt[b], n)
        pref = _torch_attention(qp[16 * b:16 * b + 16], k, v,
                                torch.arange(n - 16, n, device=dev))
        err = float((out[16 * b:16 * b + 16].float() - pref).abs().max())
        assert err <= 2e-3, (b, err)
    del dd
    torch.cuda.empty_cache()
