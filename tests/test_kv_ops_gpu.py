"""kv_ops (the reference's kv_ops_triton op) on the HIP index kernels vs the oracle:
bit-exact gather and functional scatter on contiguous and strided caches."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu


def bits(t):
    ti = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}[t.dtype]
    return t.detach().cpu().contiguous().view(ti).numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128, 12])
def test_gather_scatter(iva, dev, dtype, head_dim):
    g = torch.Generator().manual_seed(head_dim)
    kv = torch.randn(3, 5, 40, head_dim, generator=g).to(dtype)
    idx = torch.tensor([39, 0, 17, 17, 5, 22])
    out = iva.kv_ops(kv.to(dev), idx.to(dev), operation="gather")
    assert out.dtype == dtype and out.shape == (3, 5, 6, head_dim)
    assert np.array_equal(bits(out), orc.index_gather(bits(kv), idx.numpy()))
    uniq = torch.tensor([39, 0, 17, 5])
    vals = torch.randn(3, 5, 4, head_dim, generator=g).to(dtype)
    kv_dev = kv.to(dev)
    res = iva.kv_ops(kv_dev, uniq.to(dev), vals.to(dev), operation="scatter")
    assert np.array_equal(bits(res), orc.index_scatter(bits(kv), uniq.numpy(), bits(vals)))
    assert np.array_equal(bits(kv_dev), bits(kv)), "scatter must not modify its input"


def test_strided_views(iva, dev):
    """A [B, S, H, D] buffer viewed as [B, H, S, D] (transpose) and a strided values view."""
    g = torch.Generator().manual_seed(1)
    base = torch.randn(2, 30, 4, 64, generator=g).half().to(dev)
    kv = base.transpose(1, 2)
    assert not kv.is_contiguous()
    idx = torch.tensor([3, 29, 0], device=dev)
    out = iva.kv_ops(kv, idx, operation="gather")
    assert torch.equal(out.view(torch.int16), kv[:, :, idx].contiguous().view(torch.int16))
    vals = torch.randn(2, 4, 3, 128, generator=g).half().to(dev)[..., ::2]
    res = iva.kv_ops(kv, idx, vals, operation="scatter")
    ref = kv.clone()
    ref[:, :, idx] = vals
    assert torch.equal(res.view(torch.int16), ref.view(torch.int16))


def test_out_of_range_index_raises(iva, dev):
    kv = torch.zeros(1, 1, 8, 16, device=dev)
    with pytest.raises(IndexError):
        iva.kv_ops(kv, torch.tensor([8], device=dev), operation="gather")
    with pytest.raises(IndexError):
        iva.kv_ops(kv, torch.tensor([-1], device=dev), torch.zeros(1, 1, 1, 16, device=dev), "scatter")


def test_kv_ops_in_a_hip_graph(iva, dev):
    """kv_ops captured into a HIP graph (no host read of the indices then): every replay,
    with new cache contents written eagerly between replays, equals the eager op; an
    out-of-range index gathers zeros and is not scattered."""
    g = torch.Generator().manual_seed(7)
    kv = torch.randn(2, 3, 24, 64, generator=g).half().to(dev)
    idx = torch.tensor([5, 23, 0, 40, 11], device=dev)   # 40 is outside S = 24
    vals = torch.randn(2, 3, 5, 64, generator=g).half().to(dev)
    ok = torch.tensor([True, True, True, False, True], device=dev)
    iva.kv_ops(kv, idx[ok], operation="gather")          # warm-up outside the capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gathered = iva.kv_ops(kv, idx, operation="gather")
        scattered = iva.kv_ops(kv, idx, vals, operation="scatter")
    for rep in range(3):
        kv.copy_(torch.randn(2, 3, 24, 64, generator=g).half().to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = torch.zeros_like(gathered)
        want[:, :, ok] = iva.kv_ops(kv, idx[ok], operation="gather")
        assert torch.equal(gathered.view(torch.int16), want.view(torch.int16)), f"replay {rep}"
        want_s = iva.kv_ops(kv, idx[ok], vals[:, :, ok], operation="scatter")
        assert torch.equal(scattered.view(torch.int16), want_s.view(torch.int16)), f"replay {rep}"
