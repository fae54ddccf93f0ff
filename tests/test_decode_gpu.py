"""Paged decode attention on the GPU vs the fp64 CPU oracle and a torch fp32 reference.

Tolerance (written here, per the north star): max |out - exact| <= 2e-3 for fp16/bf16
and <= 1e-5 for fp32, where `exact` is the fp64 oracle.  For unit-scale test data
with peaky softmaxes the bf16/fp16 OUTPUT rounding alone can exceed that, so the
bound used in the small-shape sweeps is 2e-3 (1e-5) plus one half-ulp of the output
dtype times |exact|; the full-size config tests use the plain 2e-3 bound.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

ATOL = {torch.float16: 2e-3, torch.bfloat16: 2e-3, torch.float32: 1e-5}
OUT_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle_out(d, scale=None, window=0, n_sink=0, layout=None):
    lay = layout or d["layout"]
    return orc.decode_attention(to_np(d["q"]), to_np(d["k_pool"]), to_np(d["v_pool"]),
                                lay.block_tables.numpy(), lay.context_lens.numpy(),
                                scale=scale, window=window, n_sink=n_sink)


def run_gpu(iva, dev, d, layout=None, **kw):
    lay = layout or d["layout"]
    return iva.paged_decode_attention(d["q"].to(dev), d["k_pool"].to(dev), d["v_pool"].to(dev),
                                      lay.block_tables.to(dev), lay.context_lens.to(dev), **kw)


def assert_close(out: torch.Tensor, ref: np.ndarray, dtype, rel_ulp=True, what=""):
    err = np.abs(to_np(out) - ref)
    bound = ATOL[dtype] + (OUT_ULP[dtype] * np.abs(ref) if rel_ulp else 0.0)
    worst = float((err - bound).max()) if err.size else -1.0
    assert worst <= 0.0, f"{what}: max abs err {err.max():.3e} exceeds bound (excess {worst:.3e})"
    return float(err.max()) if err.size else 0.0


def torch_rows(k_pool, v_pool, bt_row, length):
    """Contiguous [Hkv, L, D] K/V of one sequence by plain torch indexing of the pools."""
    n = -(-length // 16)
    pages = bt_row[:n].long()
    hkv = k_pool.shape[1]
    d = k_pool.shape[2] * k_pool.shape[4]
    k = k_pool[pages].permute(1, 0, 3, 2, 4).reshape(hkv, n * 16, d)[:, :length]
    v = v_pool[pages].permute(1, 0, 3, 2).reshape(hkv, n * 16, d)[:, :length]
    return k, v


def torch_reference(q, k_pool, v_pool, bt, lengths, scale, window=0, n_sink=0):
    """fp32 torch attention on the GPU, one sequence at a time (visible keys only)."""
    batch, hq, d = q.shape
    hkv = k_pool.shape[1]
    out = torch.zeros(batch, hq, d, dtype=torch.float32, device=q.device)
    for b, length in enumerate(lengths):
        if length <= 0:
            continue
        k, v = torch_rows(k_pool, v_pool, bt[b], length)
        j = torch.arange(length, device=q.device)
        vis = (j >= length - window) | (j < n_sink) if window else torch.ones_like(j, dtype=torch.bool)
        k = k[:, vis].float().repeat_interleave(hq // hkv, dim=0).contiguous()
        v = v[:, vis].float().repeat_interleave(hq // hkv, dim=0).contiguous()
        s = torch.matmul(q[b].float().unsqueeze(1), k.transpose(1, 2).contiguous()) * scale
        out[b] = torch.matmul(torch.softmax(s, dim=-1), v).squeeze(1)
    return out


LENGTHS = [1, 15, 16, 17, 100, 257, 513, 1100]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("group", [1, 4, 16])
def test_small_vs_oracle(iva, dev, dtype, head_dim, group):
    hkv = 2
    d = iva.workloads.decode_batch(LENGTHS, hkv * group, hkv, head_dim, dtype,
                                   seed=head_dim + group, extra_pages=3)
    out = run_gpu(iva, dev, d)
    assert_close(out, oracle_out(d), dtype, what=f"{dtype} D{head_dim} G{group}")


@pytest.mark.parametrize("group", [2, 3, 5, 6, 8, 12])
def test_other_groups(iva, dev, group):
    """GQA groups other than the sweep's, powers of two or not (any group up to 16):
    stream walk and partitioned walk."""
    d = iva.workloads.decode_batch([5, 300, 999], 3 * group, 3, 128, torch.float16, seed=group,
                                   scale=128 ** -0.5)
    ref = oracle_out(d)
    assert_close(run_gpu(iva, dev, d), ref, torch.float16, rel_ulp=False, what=f"G{group}")
    assert_close(run_gpu(iva, dev, d, partition_pages=7), ref, torch.float16, rel_ulp=False,
                 what=f"G{group} partitioned")


@pytest.mark.parametrize("pp", [1, 2, 3, 5, 16, 64])
def test_partition_sizes_agree(iva, dev, pp):
    d = iva.workloads.decode_batch([700, 1, 33, 4096], 32, 8, 128, torch.float16, seed=7,
                                   scale=128 ** -0.5)
    out = run_gpu(iva, dev, d, partition_pages=pp)
    assert_close(out, oracle_out(d), torch.float16, rel_ulp=False, what=f"partition {pp}")


def test_partial_then_merge_equals_full(iva, dev):
    d = iva.workloads.decode_batch([900, 20, 2000], 16, 4, 128, torch.bfloat16, seed=8)
    lay = d["layout"]
    args = (d["q"].to(dev), d["k_pool"].to(dev), d["v_pool"].to(dev), lay.block_tables.to(dev),
            lay.context_lens.to(dev))
    # the partitioned walk in one call (explicit partition size) vs its two halves
    full = iva.paged_decode_attention(*args, partition_pages=32)
    ws = torch.empty(max(iva.decode_workspace_bytes(3, 16, 4, 128, 16, lay.block_tables.shape[1]),
                         iva.decode_workspace_bytes(3, 16, 4, 128, 16, lay.block_tables.shape[1],
                                                    partition_pages=32)),
                     dtype=torch.uint8, device=dev)
    out = torch.empty_like(full)
    iva.paged_decode_attention_partial(*args, out=out, workspace=ws, partition_pages=32)
    iva.paged_decode_attention_merge(*args, out=out, workspace=ws, partition_pages=32)
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
    # the default (stream) walk in one call vs its two halves
    full = iva.paged_decode_attention(*args)
    out = torch.empty_like(full)
    iva.paged_decode_attention_partial(*args, out=out, workspace=ws)
    iva.paged_decode_attention_merge(*args, out=out, workspace=ws)
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))


def test_deterministic(iva, dev):
    d = iva.workloads.decode_batch([4000, 37, 1500], 32, 8, 128, torch.float16, seed=9,
                                   scale=128 ** -0.5)
    a = run_gpu(iva, dev, d)
    b = run_gpu(iva, dev, d)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_closed_forms(iva, dev, dtype):
    """One key -> exactly v[0]; all keys equal -> mean of v; empty context -> zeros."""
    d = iva.workloads.decode_batch([1, 64, 0], 8, 2, 128, dtype, seed=10)
    lay = d["layout"]
    k_pool, v_pool = d["k_pool"].clone(), d["v_pool"].clone()
    # sequence 1: make all 64 keys identical (copy row 0 of its first page everywhere)
    pages = lay.block_tables[1, :4].long()
    # k_pool[p] is [Hkv, D/X, bs, X]: row 0 of the first page is [:, :, 0:1, :]
    k_pool[pages] = k_pool[pages[0]][:, :, 0:1, :].unsqueeze(0).expand_as(k_pool[pages]).clone()
    d2 = dict(d, k_pool=k_pool, v_pool=v_pool)
    out = run_gpu(iva, dev, d2).float().cpu()
    # one key: exactly the V row of position 0
    _, v0 = torch_rows(k_pool, v_pool, lay.block_tables[0], 1)
    g = 4
    for h in range(8):
        assert torch.equal(out[0, h], v0[h // g, 0].float()), "single key must return v[0] exactly"
    # equal keys: mean of the 64 V rows
    _, v1 = torch_rows(k_pool, v_pool, lay.block_tables[1], 64)
    mean = v1.double().mean(dim=1)
    for h in range(8):
        err = (out[1, h].double() - mean[h // g]).abs().max().item()
        assert err <= ATOL[dtype] + OUT_ULP[dtype] * mean[h // g].abs().max().item()
    assert not out[2].any(), "empty context must give a zero row"


@pytest.mark.parametrize("window,n_sink,lengths", [
    (64, 4, [5000, 64, 65, 63, 1]),
    (100, 0, [5000, 101, 99]),
    (16, 20, [300, 17, 40]),          # sinks reach past the window start of short sequences
    (4096, 4, [4100, 8192, 4097]),
    (1, 1, [50, 1, 2]),
])
def test_window_and_sinks(iva, dev, window, n_sink, lengths):
    d = iva.workloads.decode_batch(lengths, 8, 2, 128, torch.bfloat16, seed=window + n_sink)
    out = run_gpu(iva, dev, d, window=window, n_sink=n_sink)
    ref = oracle_out(d, window=window, n_sink=n_sink)
    assert_close(out, ref, torch.bfloat16, what=f"window {window} sinks {n_sink}")


def test_invalid_pages_are_not_attended(iva, dev):
    d = iva.workloads.decode_batch([300, 300], 8, 2, 64, torch.float32, seed=11)
    lay = d["layout"]
    bt = lay.block_tables.clone()
    bt[0, 3] = -1
    bt[1, 5] = lay.num_pages + 7
    lay2 = iva.workloads.PagedLayout(lay.lengths, bt, lay.num_pages)
    out = run_gpu(iva, dev, d, layout=lay2)
    assert_close(out, oracle_out(d, layout=lay2), torch.float32, what="invalid pages")


def test_argument_errors(iva, dev):
    d = iva.workloads.decode_batch([40], 4, 2, 128, torch.float16, seed=12)  # 3 pages
    lay = d["layout"]
    q, kp, vp = d["q"].to(dev), d["k_pool"].to(dev), d["v_pool"].to(dev)
    bt, cl = lay.block_tables.to(dev), lay.context_lens.to(dev)
    with pytest.raises(iva._abi.IvakvError, match="GQA group"):
        iva.paged_decode_attention(torch.zeros(1, 34, 128, dtype=torch.float16, device=dev),
                                   torch.zeros(1, 2, 16, 16, 8, dtype=torch.float16, device=dev),
                                   torch.zeros(1, 2, 128, 16, dtype=torch.float16, device=dev), bt, cl)
    with pytest.raises(iva._abi.IvakvError, match="head_dim"):
        iva.paged_decode_attention(torch.zeros(1, 4, 96, dtype=torch.float16, device=dev),
                                   torch.zeros(1, 2, 12, 16, 8, dtype=torch.float16, device=dev),
                                   torch.zeros(1, 2, 96, 16, dtype=torch.float16, device=dev), bt, cl)
    with pytest.raises(TypeError):
        iva.paged_decode_attention(q.float(), kp, vp, bt, cl)
    with pytest.raises(ValueError):
        iva.paged_decode_attention(q, kp, vp, bt, cl, workspace=torch.empty(1, dtype=torch.uint8, device=dev),
                                   partition_pages=1)


# ---------------------------------------------------------------- full-size configs

def test_c2_full_size(iva, dev):
    """C2: B 32, GQA 32/8, D 128, fp16, context U[512, 4096]: every sequence vs torch fp32,
    four of them vs the fp64 oracle; max abs err <= 2e-3."""
    d = iva.workloads.c2_decode(seed=0, device=dev)
    lay = d["layout"]
    bt = lay.block_tables.to(dev)
    out = iva.paged_decode_attention(d["q"], d["k_pool"], d["v_pool"], bt, lay.context_lens.to(dev))
    scale = 1 / math.sqrt(128)
    ref = torch_reference(d["q"], d["k_pool"], d["v_pool"], bt, lay.lengths, scale)
    err = (out.float() - ref).abs().max().item()
    assert err <= 2e-3, f"C2 max abs err vs torch fp32 {err}"
    pick = [0, 7, 19, 31]
    sub = iva.workloads.PagedLayout([lay.lengths[i] for i in pick], lay.block_tables[pick], lay.num_pages)
    exact = orc.decode_attention(to_np(d["q"][pick]), to_np(d["k_pool"]), to_np(d["v_pool"]),
                                 sub.block_tables.numpy(), sub.context_lens.numpy())
    err64 = float(np.abs(to_np(out[pick]) - exact).max())
    assert err64 <= 2e-3, f"C2 max abs err vs fp64 oracle {err64}"


def test_c2_fused_step_full_size(iva, dev):
    """The op bench.py times for C2, on the bench's own first pool set (c2_lengths(0),
    pools of decode_batch seed 100, new rows from a device generator seeded 500):
    paged_decode_append_attention leaves the pools bit-identical to kv_append of the new
    rows at position L-1, and its output over all 32 sequences is within the fp16
    tolerance of the fp64 oracle evaluated on the appended pools; so is the unfused
    append + attention."""
    lengths = iva.workloads.c2_lengths(seed=0)
    sc = 1 / math.sqrt(128)
    d = iva.workloads.decode_batch(lengths, 32, 8, 128, torch.float16, seed=100, device=dev,
                                   scale=sc)
    lay = d["layout"]
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    gen = torch.Generator(device=dev).manual_seed(500)
    k_new = (torch.randn(32, 8, 128, generator=gen, device=dev) * sc).half()
    v_new = (torch.randn(32, 8, 128, generator=gen, device=dev) * sc).half()
    kp_f, vp_f = d["k_pool"].clone(), d["v_pool"].clone()
    out = iva.paged_decode_append_attention(d["q"], k_new, v_new, kp_f, vp_f, bt, ctx)
    slots = torch.stack([lay.slots(b, torch.tensor([n - 1])) for b, n in enumerate(lengths)])
    kp_a, vp_a = d["k_pool"].clone(), d["v_pool"].clone()
    iva.kv_append(k_new, v_new, kp_a, vp_a, slots.reshape(-1).to(dev))
    assert torch.equal(kp_f.view(torch.int16), kp_a.view(torch.int16))
    assert torch.equal(vp_f.view(torch.int16), vp_a.view(torch.int16))
    ref = orc.decode_attention(to_np(d["q"]), to_np(kp_a), to_np(vp_a),
                               lay.block_tables.numpy(), lay.context_lens.numpy())
    err = assert_close(out, ref, torch.float16, what="C2 fused step")
    unfused = iva.paged_decode_attention(d["q"], kp_a, vp_a, bt, ctx)
    assert_close(unfused, ref, torch.float16, what="C2 append + attention")
    print(f"C2 fused step: max abs err vs fp64 oracle {err:.2e} over all 32 sequences")


def test_caller_buffers_must_be_on_the_device(iva, dev):
    """Outputs and workspaces the caller passes in are refused before any launch when
    they are on the CPU or not contiguous (the library writes through their pointers):
    decode, the fused step, prefill (both paths) and gather."""
    d = iva.workloads.decode_batch([40, 7], 8, 2, 64, torch.float16, seed=3, device=dev)
    lay = d["layout"]
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    args = (d["q"], d["k_pool"], d["v_pool"], bt, ctx)
    nbytes = iva.decode_workspace_bytes(2, 8, 2, 64, 16, bt.shape[1])
    cpu_out = torch.empty_like(d["q"], device="cpu")
    cpu_ws = torch.empty(nbytes, dtype=torch.uint8)
    strided_ws = torch.empty(2 * nbytes, dtype=torch.uint8, device=dev)[::2]
    with pytest.raises(RuntimeError, match="out is on cpu"):
        iva.paged_decode_attention(*args, out=cpu_out)
    with pytest.raises(RuntimeError, match="workspace is on cpu"):
        iva.paged_decode_attention(*args, workspace=cpu_ws)
    with pytest.raises(ValueError, match="workspace must be contiguous"):
        iva.paged_decode_attention(*args, workspace=strided_ws)
    k1 = torch.zeros(2, 2, 64, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="out is on cpu"):
        iva.paged_decode_append_attention(d["q"], k1, k1, d["k_pool"], d["v_pool"], bt, ctx,
                                          out=cpu_out)
    with pytest.raises(RuntimeError, match="workspace is on cpu"):
        iva.paged_decode_append_attention(d["q"], k1, k1, d["k_pool"], d["v_pool"], bt, ctx,
                                          workspace=cpu_ws)
    qs = torch.tensor([0, 8, 11], dtype=torch.int32, device=dev)
    qp = torch.zeros(11, 8, 64, dtype=torch.float16, device=dev)
    for split in (False, True):
        with pytest.raises(RuntimeError, match="out is on cpu"):
            iva.paged_prefill_attention(qp, d["k_pool"], d["v_pool"], bt, ctx, qs, split=split,
                                        out=torch.empty_like(qp, device="cpu"))
    pws = iva.prefill_split_workspace_bytes(2, 8, 2, 64, 8, torch.float16)
    with pytest.raises(RuntimeError, match="workspace is on cpu"):
        iva.paged_prefill_attention(qp, d["k_pool"], d["v_pool"], bt, ctx, qs, split=True,
                                    workspace=torch.empty(pws, dtype=torch.uint8))
    shape = (2, 2, 48, 64)
    with pytest.raises(RuntimeError, match="gather output is on cpu"):
        iva.kv_gather(d["k_pool"], d["v_pool"], bt, ctx, out_len=48,
                      out=(torch.empty(shape, dtype=torch.float16),
                           torch.empty(shape, dtype=torch.float16)))


@pytest.mark.parametrize("batch", [8192, 8193, 9000])
def test_batches_around_the_stream_walk_limit(iva, dev, batch):
    """Up to 8192 sequences take the stream walk, more the partitioned walk: the default
    op and the fused step at and past the switch, short contexts (empty ones included),
    checked against the fp64 oracle on 160 sequences (both ends and a random sample);
    the fused step's pools are bit-identical to kv_append of the new rows."""
    gen = torch.Generator().manual_seed(batch)
    lengths = torch.randint(0, 41, (batch,), generator=gen).tolist()
    lengths[0], lengths[-1] = 0, 40
    d = iva.workloads.decode_batch(lengths, 4, 2, 64, torch.float16, seed=batch % 97,
                                   device=dev, scale=0.125)
    lay = d["layout"]
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    pick = torch.cat([torch.arange(16), torch.arange(batch - 16, batch),
                      torch.randperm(batch - 32, generator=gen)[:128] + 16])
    bt_np, ctx_np = lay.block_tables[pick].numpy(), lay.context_lens[pick].numpy()
    out = iva.paged_decode_attention(d["q"], d["k_pool"], d["v_pool"], bt, ctx)
    ref = orc.decode_attention(to_np(d["q"][pick.to(dev)]), to_np(d["k_pool"]), to_np(d["v_pool"]),
                               bt_np, ctx_np)
    assert_close(out[pick.to(dev)], ref, torch.float16, what=f"batch {batch}")
    # the fused step: the new token at position L-1 of every non-empty sequence
    k_new = (torch.randn(batch, 2, 64, generator=gen) * 0.125).half().to(dev)
    v_new = (torch.randn(batch, 2, 64, generator=gen) * 0.125).half().to(dev)
    kp_f, vp_f = d["k_pool"].clone(), d["v_pool"].clone()
    fused = iva.paged_decode_append_attention(d["q"], k_new, v_new, kp_f, vp_f, bt, ctx)
    slots = torch.tensor([int(lay.slots(b, torch.tensor([n - 1]))[0]) if n > 0 else -1
                          for b, n in enumerate(lengths)], dtype=torch.int32)
    kp_a, vp_a = d["k_pool"].clone(), d["v_pool"].clone()
    iva.kv_append(k_new, v_new, kp_a, vp_a, slots.to(dev))
    assert torch.equal(kp_f.view(torch.int16), kp_a.view(torch.int16))
    assert torch.equal(vp_f.view(torch.int16), vp_a.view(torch.int16))
    ref = orc.decode_attention(to_np(d["q"][pick.to(dev)]), to_np(kp_a), to_np(vp_a), bt_np, ctx_np)
    assert_close(fused[pick.to(dev)], ref, torch.float16, what=f"fused batch {batch}")


def test_c4_long_context(iva, dev):
    """C4: B 4 at 32k..128k tokens, window 4096 + 4 sinks, bf16, K/V ~ N(0,1)."""
    d = iva.workloads.c4_long_context(seed=0, device=dev)
    lay = d["layout"]
    bt = lay.block_tables.to(dev)
    out = iva.paged_decode_attention(d["q"], d["k_pool"], d["v_pool"], bt, lay.context_lens.to(dev),
                                     window=d["window"], n_sink=d["n_sink"])
    ref = torch_reference(d["q"], d["k_pool"], d["v_pool"], bt, lay.lengths, 1 / math.sqrt(128),
                          window=d["window"], n_sink=d["n_sink"])
    err = (out.float() - ref).abs().max().item()
    assert err <= 2e-3, f"C4 max abs err {err}"


def test_c5_ragged(iva, dev):
    """C5 shapes: 256 ragged sequences (LogNormal median 1024, sigma 1, cap 16k), fp16."""
    lengths = iva.workloads.c5_lengths(seed=0)
    d = iva.workloads.decode_batch(lengths, 32, 8, 128, torch.float16, seed=5, device=dev,
                                   scale=128 ** -0.5)
    lay = d["layout"]
    bt = lay.block_tables.to(dev)
    out = iva.paged_decode_attention(d["q"], d["k_pool"], d["v_pool"], bt, lay.context_lens.to(dev))
    ref = torch_reference(d["q"], d["k_pool"], d["v_pool"], bt, lay.lengths, 1 / math.sqrt(128))
    err = (out.float() - ref).abs().max().item()
    assert err <= 2e-3, f"C5 max abs err {err}"


def test_golden_tiny_fixture(iva, dev):
    """tests/golden/decode_tiny.npz: fp32, GQA 4/2, head_dim 8 is below the kernel's minimum
    head_dim, so the fixture's rows are zero-padded to 64 dims (padding changes no score
    and no output column); expected values were evaluated term by term in pure Python."""
    from pathlib import Path
    g = np.load(Path(__file__).resolve().parent / "golden" / "decode_tiny.npz")
    kp8, vp8 = g["k_pool"], g["v_pool"]            # [P, 2, 2, 16, 4], [P, 2, 8, 16]
    p, h = kp8.shape[:2]
    kp = np.zeros((p, h, 16, 16, 4), np.float32)
    kp[:, :, :2] = kp8
    vp = np.zeros((p, h, 64, 16), np.float32)
    vp[:, :, :8] = vp8
    q = np.zeros((2, 4, 64), np.float32)
    q[:, :, :8] = g["q"]
    out = iva.paged_decode_attention(torch.from_numpy(q).to(dev), torch.from_numpy(kp).to(dev),
                                     torch.from_numpy(vp).to(dev),
                                     torch.from_numpy(g["block_tables"]).to(dev),
                                     torch.from_numpy(g["context_lens"]).to(dev),
                                     scale=1 / math.sqrt(8), window=int(g["window"]),
                                     n_sink=int(g["n_sink"]))
    err = np.abs(to_np(out)[:, :, :8] - g["expected"]).max()
    assert err <= 1e-5, f"golden fixture max abs err {err}"
    assert not to_np(out)[:, :, 8:].any()


def test_context_beyond_block_table(iva, dev):
    """context_lens larger than the block table can address: positions past the table are
    not attended (and no partition reaches past the workspace)."""
    d = iva.workloads.decode_batch([300, 40], 8, 2, 128, torch.float16, seed=13, scale=128 ** -0.5)
    lay = d["layout"]
    lay2 = iva.workloads.PagedLayout([300 + 5000, 40], lay.block_tables, lay.num_pages)
    out = run_gpu(iva, dev, d, layout=lay2)
    assert_close(out, oracle_out(d, layout=lay2), torch.float16, rel_ulp=False, what="ctx > table")
    out_w = run_gpu(iva, dev, d, layout=lay2, window=200, n_sink=4)
    assert_close(out_w, oracle_out(d, layout=lay2, window=200, n_sink=4), torch.float16,
                 rel_ulp=False, what="ctx > table, window")



def test_workspace_reuse_across_calls(iva, dev):
    """One workspace, filled with garbage (it needs no initialisation), serves alternating
    batches of different shapes through both walks (stream walk and 8-page partitions);
    results stay exact."""
    a = iva.workloads.decode_batch([3000, 700, 16, 2500], 32, 8, 128, torch.float16, seed=21,
                                   scale=128 ** -0.5)
    b = iva.workloads.decode_batch([900, 4000], 32, 8, 128, torch.float16, seed=22,
                                   scale=128 ** -0.5)
    need = max(iva.decode_workspace_bytes(len(d["lengths"]), 32, 8, 128, 16,
                                          d["layout"].block_tables.shape[1], partition_pages=pp)
               for d in (a, b) for pp in (0, 8))
    ws = torch.full((need,), 0x7F, dtype=torch.uint8, device=dev)
    for _ in range(3):
        for d, pp in ((a, 8), (b, 0), (a, 0), (b, 8)):
            out = run_gpu(iva, dev, d, workspace=ws, partition_pages=pp)
            assert_close(out, oracle_out(d), torch.float16, rel_ulp=False,
                         what=f"workspace reuse, partition_pages {pp}")


@pytest.mark.parametrize("lengths", [
    [0, 0, 5, 0, 4097, 0, 1, 16, 17, 0],        # empty sequences between long and tiny ones
    [1],                                        # fewer tiles than a wave minimum
    [16] * 300,                                 # many one-page units: waves span many units
    [3000, 2, 2, 2, 2, 2, 2, 2, 2, 2999],       # units split across many waves next to tiny ones
])
def test_stream_walk_unit_boundaries(iva, dev, lengths):
    """The default (stream) walk against the oracle where wave ranges cross many unit
    boundaries, units are empty, or the batch is smaller than one wave's share."""
    d = iva.workloads.decode_batch(lengths, 16, 4, 128, torch.float16, seed=len(lengths),
                                   scale=128 ** -0.5, extra_pages=2)
    out = run_gpu(iva, dev, d)
    assert_close(out, oracle_out(d), torch.float16, rel_ulp=False, what=f"stream {lengths[:4]}")


def test_stream_matches_partitioned(iva, dev):
    """Stream and partitioned walks agree on a C5-like ragged batch (fp16 tolerance)."""
    lengths = iva.workloads.c5_lengths(seed=3, n_seqs=64)
    d = iva.workloads.decode_batch(lengths, 32, 8, 128, torch.float16, seed=31, device=dev,
                                   scale=128 ** -0.5)
    lay = d["layout"]
    args = (d["q"], d["k_pool"], d["v_pool"], lay.block_tables.to(dev), lay.context_lens.to(dev))
    a = iva.paged_decode_attention(*args)
    b = iva.paged_decode_attention(*args, partition_pages=24)
    assert (a.float() - b.float()).abs().max().item() <= 2e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("window,n_sink", [(0, 0), (40, 4)])
def test_fused_append_attention(iva, dev, dtype, window, n_sink):
    """ivakv_decode_append_attn == ivakv_append of the new rows + ivakv_decode_attn: the
    pools afterwards are bit-identical, the output matches the fp64 oracle (tolerance of
    the dtype).  Lengths cover a new token alone (L=1), an empty sequence (L=0), a new
    token opening a page (L=17) and closing one (L=16), and an invalid page id under
    the new token (neither stored nor attended)."""
    lengths = [1, 0, 17, 16, 300, 1000, 2]
    hkv, g, d = 2, 4, 128
    base = iva.workloads.decode_batch(lengths, hkv * g, hkv, d, dtype, seed=40 + window,
                                      scale=0.5, extra_pages=4)
    lay = base["layout"]
    bt = lay.block_tables.clone()
    bt[6, 0] = -3                      # the new token of sequence 6 sits on an invalid page
    lay = iva.workloads.PagedLayout(lay.lengths, bt, lay.num_pages)
    gen = torch.Generator().manual_seed(7)
    k_new = (torch.randn(len(lengths), hkv, d, generator=gen) * 0.5).to(dtype)
    v_new = (torch.randn(len(lengths), hkv, d, generator=gen) * 0.5).to(dtype)
    # reference: append then decode
    kp_a, vp_a = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    slots = torch.tensor([int(bt[b, (n - 1) // 16]) * 16 + (n - 1) % 16 if n > 0 and bt[b, (n - 1) // 16] >= 0
                          else -1 for b, n in enumerate(lengths)], dtype=torch.int32)
    iva.kv_append(k_new.to(dev), v_new.to(dev), kp_a, vp_a, slots.to(dev))
    # fused
    kp_f, vp_f = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    out = iva.paged_decode_append_attention(base["q"].to(dev), k_new.to(dev), v_new.to(dev), kp_f,
                                            vp_f, lay.block_tables.to(dev), lay.context_lens.to(dev),
                                            window=window, n_sink=n_sink)
    ti = {torch.float32: torch.int32}.get(dtype, torch.int16)
    assert torch.equal(kp_a.view(ti), kp_f.view(ti)) and torch.equal(vp_a.view(ti), vp_f.view(ti))
    d_after = dict(base, k_pool=kp_a.cpu(), v_pool=vp_a.cpu())
    ref = oracle_out(d_after, window=window, n_sink=n_sink, layout=lay)
    assert_close(out, ref, dtype, what=f"fused {dtype} w{window}")
    unfused = iva.paged_decode_attention(base["q"].to(dev), kp_a, vp_a, lay.block_tables.to(dev),
                                         lay.context_lens.to(dev), window=window, n_sink=n_sink)
    assert_close(unfused, ref, dtype, what="append + decode")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("window,n_sink", [(0, 0), (100, 4)])
def test_fused_one_partition_per_sequence(iva, dev, dtype, d, window, n_sink):
    """Batches with at least one (sequence, kv head) unit per CU whose tables hold at
    most 64 pages run the fused op on one partition per sequence (a workgroup per unit,
    its waves merged in LDS, the new token folded in, no merge kernel): 128 ragged
    sequences of up to 1000 tokens x 4 kv heads, with a new token alone (L=1), an empty
    sequence, a new token opening and closing a page, and an invalid page id under a
    new token.  Pools bit-identical to append + decode, output within the dtype's
    tolerance of the fp64 oracle."""
    gen = torch.Generator().manual_seed(23 + d)
    lengths = [1, 0, 17, 16, 1000, 2, 33] + torch.randint(0, 1000, (121,), generator=gen).tolist()
    hkv, g = 4, 4
    base = iva.workloads.decode_batch(lengths, hkv * g, hkv, d, dtype, seed=70 + d,
                                      scale=d ** -0.5, extra_pages=4)
    lay = base["layout"]
    assert lay.block_tables.shape[1] <= 64
    bt = lay.block_tables.clone()
    bt[6, 2] = -1                      # the new token of sequence 6 (L=33) sits on an invalid page
    lay = iva.workloads.PagedLayout(lay.lengths, bt, lay.num_pages)
    k_new = (torch.randn(len(lengths), hkv, d, generator=gen) * d ** -0.5).to(dtype)
    v_new = (torch.randn(len(lengths), hkv, d, generator=gen) * d ** -0.5).to(dtype)
    kp_a, vp_a = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    slots = torch.tensor([int(bt[b, (n - 1) // 16]) * 16 + (n - 1) % 16
                          if n > 0 and bt[b, (n - 1) // 16] >= 0 else -1
                          for b, n in enumerate(lengths)], dtype=torch.int32)
    iva.kv_append(k_new.to(dev), v_new.to(dev), kp_a, vp_a, slots.to(dev))
    kp_f, vp_f = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    out = iva.paged_decode_append_attention(base["q"].to(dev), k_new.to(dev), v_new.to(dev), kp_f,
                                            vp_f, bt.to(dev), lay.context_lens.to(dev),
                                            window=window, n_sink=n_sink)
    ti = {torch.float32: torch.int32}.get(dtype, torch.int16)
    assert torch.equal(kp_a.view(ti), kp_f.view(ti)) and torch.equal(vp_a.view(ti), vp_f.view(ti))
    ref = oracle_out(dict(base, k_pool=kp_a.cpu(), v_pool=vp_a.cpu()), window=window,
                     n_sink=n_sink, layout=lay)
    assert_close(out, ref, dtype, what=f"fused one partition d{d} w{window}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_many_units_merges(iva, dev, dtype, d):
    """Batches of >= 1024 (sequence, kv head) units take the merges with four output
    elements per thread (the fused op's new-token dot product then sums over the D/4
    lanes of a head): 160 short ragged sequences x 8 kv heads, one of 1100 tokens so
    that the table is wider than one partition's limit and the fused op keeps the
    stream walk.  Fused op: pools bit-identical to append + decode; both outputs within
    the dtype's tolerance of the fp64 oracle."""
    gen = torch.Generator().manual_seed(11)
    lengths = [1, 0, 17, 16, 1100, 2] + torch.randint(0, 80, (154,), generator=gen).tolist()
    hkv, g = 8, 4
    base = iva.workloads.decode_batch(lengths, hkv * g, hkv, d, dtype, seed=60 + d,
                                      scale=d ** -0.5, extra_pages=4)
    lay = base["layout"]
    bt = lay.block_tables
    k_new = (torch.randn(len(lengths), hkv, d, generator=gen) * d ** -0.5).to(dtype)
    v_new = (torch.randn(len(lengths), hkv, d, generator=gen) * d ** -0.5).to(dtype)
    kp_a, vp_a = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    slots = torch.tensor([int(bt[b, (n - 1) // 16]) * 16 + (n - 1) % 16 if n > 0 else -1
                          for b, n in enumerate(lengths)], dtype=torch.int32)
    iva.kv_append(k_new.to(dev), v_new.to(dev), kp_a, vp_a, slots.to(dev))
    kp_f, vp_f = base["k_pool"].clone().to(dev), base["v_pool"].clone().to(dev)
    out = iva.paged_decode_append_attention(base["q"].to(dev), k_new.to(dev), v_new.to(dev), kp_f,
                                            vp_f, bt.to(dev), lay.context_lens.to(dev))
    assert torch.equal(kp_a.view(torch.int16), kp_f.view(torch.int16))
    assert torch.equal(vp_a.view(torch.int16), vp_f.view(torch.int16))
    ref = oracle_out(dict(base, k_pool=kp_a.cpu(), v_pool=vp_a.cpu()))
    assert_close(out, ref, dtype, what=f"fused many units d{d}")
    unfused = iva.paged_decode_attention(base["q"].to(dev), kp_a, vp_a, bt.to(dev),
                                         lay.context_lens.to(dev))
    assert_close(unfused, ref, dtype, what=f"stream merge many units d{d}")
