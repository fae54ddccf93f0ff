"""RoPE fused into the append, query rotation, page moves, pool compaction and the
contiguous-cache compaction op on the GPU.

  * ivakv_rope / ivakv_append_rope vs the fp64 oracle (rope_kv.py:22-50): fp16 / bf16
    elements within one unit in the last place of the exactly rounded result; fp32
    within 4 ulp of the pair's magnitude (a rotated element can cancel to near zero,
    so its own ulp is no yardstick); positions up to 100k; V rows of the append and
    every untouched slot bit-exact;
  * ivakv_copy_pages and PagedKVPool.compact: bit-exact page contents (fp16 and FP8
    with scaling factors); gathered sequences identical before and after;
  * kv_compact vs torch indexing, bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu


def ulp_diff(got: torch.Tensor, exact: np.ndarray, dtype) -> float:
    """Max |got - exact| in units of the last place of the element type at |exact|."""
    ref = torch.from_numpy(exact).to(dtype).float()                 # exactly rounded
    g = got.float().cpu()
    e = torch.from_numpy(exact).float()
    mant = {torch.float16: 10, torch.bfloat16: 7, torch.float32: 23}[dtype]
    expo = torch.floor(torch.log2(torch.clamp(e.abs(), min=2.0 ** -14)))
    ulp = torch.pow(2.0, expo - mant)
    return float(((g - ref).abs() / ulp).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("d", [64, 128])
def test_rope_in_place_vs_oracle(iva, dev, dtype, d):
    g = torch.Generator().manual_seed(d)
    x = torch.randn(50, 6, d, generator=g).to(dtype)
    pos = torch.randint(0, 100000, (50,), generator=g, dtype=torch.int32)
    pos[:3] = torch.tensor([0, 1, 65535], dtype=torch.int32)
    y = iva.rope_(x.clone().to(dev), pos.to(dev), theta=10000.0)
    exact = orc.rope(x.float().numpy(), pos.numpy(), 10000.0)
    if dtype == torch.float32:
        xn = x.numpy()
        mag = np.repeat(np.hypot(xn[..., 0::2], xn[..., 1::2]), 2, axis=-1)
        assert (np.abs(y.cpu().numpy() - exact) <= 4 * 2.0 ** -23 * mag + 1e-30).all()
    else:
        assert ulp_diff(y, exact, dtype) <= 1
    assert torch.equal(y[0].cpu(), x[0])                           # position 0: identity


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("hkv,d", [(8, 64), (3, 128), (5, 64), (1, 128), (6, 256), (12, 64)])
@pytest.mark.parametrize("shift", [0, 1], ids=["aligned", "shifted"])
def test_append_rope_vs_oracle(iva, dev, dtype, hkv, d, shift):
    """Lanes rotate groups of up to eight kv heads: head counts that are not a multiple
    of eight leave a partial last group.  A row with slot -1 and one past the pool are
    skipped (pools keep the fill value).  Source rows shifted by one element are not
    16-byte aligned and take the element-wise path; aligned rows move 16-byte chunks."""
    lengths = [7, 33, 20]
    lay = iva.workloads.permuted_layout(lengths, 12, torch.Generator().manual_seed(3))
    n = sum(lengths)
    gen = torch.Generator().manual_seed(2 + hkv)
    k_new = torch.randn(n, hkv, d, generator=gen).to(dtype)
    v_new = torch.randn(n, hkv, d, generator=gen).to(dtype)
    slots = torch.cat([lay.slots(b, torch.arange(m)) for b, m in enumerate(lengths)])
    slots[5], slots[40] = -1, 12 * 16 + 3
    k_src, v_src = k_new.to(dev), v_new.to(dev)
    if shift:   # views starting one element into a wider buffer
        kb = torch.zeros(n, hkv, d + 8, dtype=dtype, device=dev)
        vb = torch.zeros(n, hkv, d + 8, dtype=dtype, device=dev)
        k_src, v_src = kb[..., 1:d + 1], vb[..., 1:d + 1]
        k_src.copy_(k_new.to(dev))
        v_src.copy_(v_new.to(dev))
        assert k_src.data_ptr() % 16 and v_src.data_ptr() % 16
    positions = torch.cat([torch.arange(m) + 1000 * b for b, m in enumerate(lengths)]).to(torch.int32)
    ks, vs = iva.pool_shapes(12, hkv, d, 16, dtype)
    kp = torch.full(ks, 3.0, dtype=dtype, device=dev)
    vp = torch.full(vs, 3.0, dtype=dtype, device=dev)
    iva.kv_append(k_src, v_src, kp, vp, slots.to(dev),
                  rope_positions=positions.to(dev), rope_theta=10000.0)
    # expected pools: the oracle append of the rotated K rows (rounded once), V as is
    k_rot = orc.rope(k_new.float().numpy(), positions.numpy(), 10000.0)
    ek = np.full(ks, 3.0)  # fp64 values in the pools' layout
    ev = np.full(vs, 3.0)
    orc.append(ek, ev, k_rot, v_new.float().numpy(), slots.numpy())
    if dtype == torch.float32:  # 4 ulp of the pair's magnitude, as for ivakv_rope
        kn = k_new.numpy()
        mag = np.full(ks, 0.0)
        orc.append(mag, np.full(vs, 0.0), np.repeat(np.hypot(kn[..., 0::2], kn[..., 1::2]), 2, -1),
                   v_new.numpy(), slots.numpy())
        assert (np.abs(kp.cpu().numpy() - ek) <= 4 * 2.0 ** -23 * mag + 1e-30).all()
    else:
        assert ulp_diff(kp, ek, dtype) <= 1
    assert torch.equal(vp.cpu(), torch.from_numpy(ev).to(dtype))


@pytest.mark.parametrize("fp8", [False, True])
def test_copy_pages_and_pool_compaction(iva, dev, fp8):
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    dtype = torch.float8_e4m3fn if fp8 else torch.float16
    pool = pc.PagedKVPool(48, 2, 64, 16, num_layers=2, dtype=dtype, device=dev, max_seqs=16)
    rng = np.random.default_rng(5)
    live = []
    for step in range(30):
        sid = ("s", step)
        pool.add_sequence(sid)
        n = int(rng.integers(1, 70))
        slots = torch.from_numpy(pool.allocate(sid, n)).to(dev)
        for layer in range(2):
            rows = torch.randn(n, 2, 64, device=dev).to(torch.float16)
            iva.kv_append(rows, rows * 2, pool.k_pools[layer], pool.v_pools[layer], slots,
                          **pool.scales(layer))
        live.append(sid)
        if len(live) > 4:
            pool.free(live.pop(int(rng.integers(len(live)))))
        if pool.num_free_pages < 10:
            break

    def gathered():
        bt, ctx = pool.device_tables(live)
        kw = {"out_dtype": torch.float16} if fp8 else {}
        return [iva.kv_gather(pool.k_pools[l], pool.v_pools[l], bt, ctx, **pool.scales(l), **kw)
                for l in range(2)]

    before = gathered()
    raw = [t.clone().view(torch.uint8).cpu() for t in pool.k_pools + pool.v_pools + pool.k_scales + pool.v_scales]
    src, dst = pool.compaction_moves()
    assert src, "the churn above must leave gaps"
    assert pool.compact() == len(src)
    after = gathered()
    for (k0, v0), (k1, v1) in zip(before, after):
        assert torch.equal(k0.view(torch.int16), k1.view(torch.int16))
        assert torch.equal(v0.view(torch.int16), v1.view(torch.int16))
    # the moved pages are byte copies; pages that did not move are untouched
    now = [t.view(torch.uint8).cpu() for t in pool.k_pools + pool.v_pools + pool.k_scales + pool.v_scales]
    for r, w in zip(raw, now):
        for s_, d_ in zip(src, dst):
            assert torch.equal(w[d_], r[s_])
        keep = [p for p in range(48) if p not in dst]
        assert torch.equal(w[keep], r[keep])


def test_copy_pages_rejects_and_skips_ids_outside_the_pool(iva, dev):
    """ops.copy_pages raises IndexError for an id outside [0, num_pages); at the C ABI
    (no host check) the kernel skips such a move and performs the others."""
    ks, vs = iva.pool_shapes(8, 2, 64, 16, torch.float16)
    k = torch.randn(ks, device=dev).half()
    v = torch.randn(vs, device=dev).half()
    k0, v0 = k.clone(), v.clone()
    for src, dst in (([1, 8], [2, 3]), ([1, 2], [-1, 3])):
        with pytest.raises(IndexError, match="outside the pool"):
            iva.copy_pages(k, v, torch.tensor(src, dtype=torch.int32, device=dev),
                           torch.tensor(dst, dtype=torch.int32, device=dev))
    assert torch.equal(k, k0) and torch.equal(v, v0)
    src = torch.tensor([1, 9, 5, 2], dtype=torch.int32, device=dev)
    dst = torch.tensor([0, 3, -2, 6], dtype=torch.int32, device=dev)
    iva._abi.call("ivakv_copy_pages", k.data_ptr(), v.data_ptr(), None, None, src.data_ptr(),
                  dst.data_ptr(), 4, 8, 2, 64, 16, 2, torch.cuda.current_stream().cuda_stream)
    want_k, want_v = k0.clone(), v0.clone()
    want_k[[0, 6]] = k0[[1, 2]]
    want_v[[0, 6]] = v0[[1, 2]]
    assert torch.equal(k, want_k) and torch.equal(v, want_v)


def test_kv_compact_vs_torch(iva, dev):
    kv = torch.randn(3, 4, 40, 64, device=dev).half()
    mask = torch.zeros(40, dtype=torch.bool)
    mask[[0, 3, 4, 17, 39]] = True
    got = iva.kv_compact(kv, mask.to(dev))
    assert torch.equal(got, kv[:, :, mask.to(dev)])
    got2 = iva.kv_compact(kv, mask.expand(3, 40).to(dev))
    assert torch.equal(got2, got)
    bad = mask.expand(3, 40).clone()
    bad[1, 5] = True
    with pytest.raises(ValueError, match="same mask"):
        iva.kv_compact(kv, bad.to(dev))


def test_copy_pages_in_a_hip_graph(iva, dev):
    """copy_pages captured into a HIP graph (no host read of the ids then): every replay,
    from pools reset eagerly between replays, equals the eager moves; a move with an id
    outside the pool is skipped by the kernel."""
    ks, vs = iva.pool_shapes(16, 2, 64, 16, torch.float16)
    k = torch.randn(ks, device=dev).half()
    v = torch.randn(vs, device=dev).half()
    src = torch.tensor([3, 7, 12, 1], dtype=torch.int32, device=dev)
    dst = torch.tensor([0, 5, 20, 9], dtype=torch.int32, device=dev)   # 20 is outside
    iva.copy_pages(k, v, src[[0, 1, 3]], dst[[0, 1, 3]])               # warm-up, eager
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        iva.copy_pages(k, v, src, dst)
    for rep in range(3):
        k0 = torch.randn(ks, device=dev).half()
        v0 = torch.randn(vs, device=dev).half()
        k.copy_(k0)
        v.copy_(v0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_k, want_v = k0.clone(), v0.clone()
        want_k[[0, 5, 9]] = k0[[3, 7, 1]]
        want_v[[0, 5, 9]] = v0[[3, 7, 1]]
        assert torch.equal(k, want_k) and torch.equal(v, want_v), f"replay {rep}"


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
def test_append_rope_fp8_equals_rope_then_append(iva, dev, src, d):
    """ivakv_append_rope_fp8 (kv_append with rope_positions on FP8 pools): codes and
    factors byte-identical to ivakv_rope on the K rows followed by the FP8 append (every
    byte of both pools and both factor tables compared), with a skipped slot and one
    outside the pool; and the dequantized K within the FP8 quantization step of the
    oracle's rotation of the source rows."""
    FP8 = torch.float8_e4m3fn
    lengths = [7, 33, 20]
    hkv = 3
    lay = iva.workloads.permuted_layout(lengths, 12, torch.Generator().manual_seed(4))
    n = sum(lengths)
    gen = torch.Generator().manual_seed(d)
    k_new = torch.randn(n, hkv, d, generator=gen).to(src)
    v_new = torch.randn(n, hkv, d, generator=gen).to(src)
    slots = torch.cat([lay.slots(b, torch.arange(m)) for b, m in enumerate(lengths)])
    slots[5], slots[40] = -1, 12 * 16 + 3
    pos = torch.cat([torch.arange(m) + 5000 * b for b, m in enumerate(lengths)]).to(torch.int32)
    ks, vs = iva.pool_shapes(12, hkv, d, 16, FP8)
    pools = []
    for fused in (True, False):
        kp = torch.full(ks, 7, dtype=torch.uint8, device=dev).view(FP8)
        vp = torch.full(vs, 7, dtype=torch.uint8, device=dev).view(FP8)
        ksc = torch.full(iva.scale_shape(12, hkv), 2.0, device=dev)
        vsc = torch.full(iva.scale_shape(12, hkv), 2.0, device=dev)
        if fused:
            iva.kv_append(k_new.to(dev), v_new.to(dev), kp, vp, slots.to(dev), k_scale=ksc,
                          v_scale=vsc, rope_positions=pos.to(dev), rope_theta=10000.0)
        else:
            k_rot = iva.rope_(k_new.to(dev).clone(), pos.to(dev), theta=10000.0)
            iva.kv_append(k_rot, v_new.to(dev), kp, vp, slots.to(dev), k_scale=ksc, v_scale=vsc)
        pools.append([t.view(torch.uint8).cpu() if t.dtype == FP8 else t.cpu() for t in (kp, vp, ksc, vsc)])
    for a, b in zip(*pools):
        assert torch.equal(a, b)
    # against the oracle: dequantized K rows within one e4m3 step (2^-3 relative) of the
    # exact rotation, plus the source dtype's rounding of the rotated value
    kd, vd = orc.dequantize_pools(pools[0][0].numpy(), pools[0][1].numpy(), pools[0][2].numpy(),
                                  pools[0][3].numpy(), np.float64)
    exact = orc.rope(k_new.float().numpy(), pos.numpy(), 10000.0)
    got = orc.gather(kd, vd, lay.block_tables.numpy(), lay.context_lens.numpy(),
                     out_len=max(lengths))[0]
    t = 0
    for b, m in enumerate(lengths):
        for i in range(m):
            if t + i in (5, 40):
                continue
            row, ref = got[b, :, i], exact[t + i]
            amax = np.abs(ref).max(axis=-1, keepdims=True)
            assert (np.abs(row - ref) <= 2.0 ** -4 * np.maximum(np.abs(ref), amax / 64) + 1e-6).all()
        t += m
