"""Host threads on separate streams: each stream gets its own op-owned workspace, so decode
attention, the fused step and the split prefill launched concurrently from four threads
give the same bits as one thread alone (all three are deterministic)."""
from __future__ import annotations

import threading

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_threads_on_separate_streams(iva, dev):
    d = iva.workloads.decode_batch([900, 3000, 17, 2500], 16, 4, 128, torch.float16, seed=51,
                                   device=dev, scale=128 ** -0.5)
    lay = d["layout"]
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    gen = torch.Generator().manual_seed(52)
    k1 = (torch.randn(4, 4, 128, generator=gen) * 0.1).half().to(dev)
    v1 = (torch.randn(4, 4, 128, generator=gen) * 0.1).half().to(dev)
    qs = torch.tensor([0, 64, 192, 209, 509], dtype=torch.int32, device=dev)
    qp = (torch.randn(509, 16, 128, generator=gen) * 0.5).half().to(dev)

    def step(kp, vp):
        dec = iva.paged_decode_attention(d["q"], kp, vp, bt, ctx)
        fused = iva.paged_decode_append_attention(d["q"], k1, v1, kp, vp, bt, ctx)
        pre = iva.paged_prefill_attention(qp, kp, vp, bt, ctx, qs, split=True, max_query_len=300)
        return dec, fused, pre

    # the fused step writes k1 / v1 at position L-1; once they are there, every op below
    # reads the same pools on every call
    iva.paged_decode_append_attention(d["q"], k1, v1, d["k_pool"], d["v_pool"], bt, ctx)
    ref = step(d["k_pool"].clone(), d["v_pool"].clone())
    torch.cuda.synchronize(dev)
    errors = []
    start = threading.Barrier(4)

    def worker(i):
        try:
            s = torch.cuda.Stream(device=dev)
            kp, vp = d["k_pool"].clone(), d["v_pool"].clone()  # each thread's own pools
            torch.cuda.synchronize(dev)
            start.wait()
            with torch.cuda.stream(s):
                for it in range(8):
                    out = step(kp, vp)
                    s.synchronize()
                    for name, a, b in zip(("decode", "fused", "prefill"), out, ref):
                        if not torch.equal(a.view(torch.int16), b.view(torch.int16)):
                            errors.append((i, it, name))
        except Exception as e:  # surfaced below
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:4]
