"""Continuous-batching churn (config C5 semantics) on fragmented block tables: sequences
start with chunked prefill appends, all live sequences take one decode append per step,
random completions return pages to the LIFO free list and new sequences reuse them.
At the end every sequence's gathered K/V is bit-exact against a host shadow of the
appended rows, and decode attention matches the fp64 oracle (fp16 bound 2e-3)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu


def test_churn_fragmented_tables(iva, dev):
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    hkv, d = 4, 128
    pool = pc.PagedKVPool(400, hkv, d, 16, 1, torch.float16, dev, max_seqs=48, max_blocks_per_seq=64)
    g = torch.Generator().manual_seed(0)
    rng = np.random.default_rng(0)
    shadow = {}
    nxt = 0

    def append(sid, n):
        k = (torch.randn(n, hkv, d, generator=g) * 0.1).half()
        v = (torch.randn(n, hkv, d, generator=g) * 0.1).half()
        slots = torch.from_numpy(pool.allocate(sid, n))
        iva.kv_append(k.to(dev), v.to(dev), pool.k_pools[0], pool.v_pools[0], slots.to(dev))
        ks, vs = shadow[sid]
        shadow[sid] = (torch.cat([ks, k]), torch.cat([vs, v]))

    def start():
        nonlocal nxt
        sid = ("s", nxt)
        nxt += 1
        pool.add_sequence(sid)
        shadow[sid] = (torch.empty(0, hkv, d).half(), torch.empty(0, hkv, d).half())
        prompt = int(rng.integers(1, 300))
        for off in range(0, prompt, 64):         # prefill chunks
            append(sid, min(64, prompt - off))

    for _ in range(24):
        start()
    for step in range(40):
        for sid in list(shadow):
            append(sid, 1)
        for sid in list(shadow):
            if rng.random() < 0.08:              # random completion
                pool.free(sid)
                del shadow[sid]
        while len(shadow) < 24:
            start()
    ids = list(shadow)
    bt, ctx = pool.device_tables(ids)
    assert (np.diff(bt.cpu().numpy()[:, :4], axis=1) != 1).any(), "tables should be fragmented"
    ko, vo = iva.kv_gather(pool.k_pools[0], pool.v_pools[0], bt, ctx)
    for i, sid in enumerate(ids):
        ks, vs = shadow[sid]
        n = ks.shape[0]
        assert torch.equal(ko[i, :, :n].cpu().view(torch.int16), ks.transpose(0, 1).contiguous().view(torch.int16))
        assert torch.equal(vo[i, :, :n].cpu().view(torch.int16), vs.transpose(0, 1).contiguous().view(torch.int16))
    q = (torch.randn(len(ids), 4 * hkv, d, generator=g) * 0.3).half()
    out = iva.paged_decode_attention(q.to(dev), pool.k_pools[0], pool.v_pools[0], bt, ctx)
    ref = orc.decode_attention(q.float().numpy(), pool.k_pools[0].float().cpu().numpy(),
                               pool.v_pools[0].float().cpu().numpy(), bt.cpu().numpy(),
                               ctx.cpu().numpy())
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= 2e-3
