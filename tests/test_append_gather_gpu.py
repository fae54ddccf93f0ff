"""Paged append / gather on the GPU vs the CPU oracle: bit-exact on bit views.

Covers config C1 (4 sequences {17, 64, 129, 200}, Hkv 8, D 64, block 16, fp32)
in all three dtypes, plus the edge cases of the reference's KV ops: empty
inputs, skipped (-1) and out-of-range slots, invalid page ids, strided and
misaligned sources, truncated/padded gathers, other block sizes and head dims,
and a 512-token prefill-chunk append.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
BITS = {torch.float32: (torch.int32, np.uint32), torch.float16: (torch.int16, np.uint16),
        torch.bfloat16: (torch.int16, np.uint16)}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a tensor as an unsigned numpy array (exact for any float dtype)."""
    ti, npu = BITS[t.dtype]
    return t.detach().cpu().contiguous().view(ti).numpy().view(npu)


def new_pools(iva, dev, num_pages, hkv, d, bs, dtype, canary=None):
    ks, vs = iva.pool_shapes(num_pages, hkv, d, bs, dtype)
    if canary is None:
        return torch.zeros(ks, dtype=dtype, device=dev), torch.zeros(vs, dtype=dtype, device=dev)
    ti, _ = BITS[dtype]
    k = torch.full(ks, canary, dtype=ti, device=dev).view(dtype)
    v = torch.full(vs, canary, dtype=ti, device=dev).view(dtype)
    return k, v


def oracle_pools(num_pages, hkv, d, bs, dtype, canary=None):
    _, npu = BITS[dtype]
    return orc.empty_pools(num_pages, hkv, d, bs, npu, fill=0 if canary is None else canary)


def run_case(iva, dev, k_new, v_new, slots, layout, num_pages, hkv, d, bs, dtype, canary=None,
             out_len=None):
    """Appends on GPU and in the oracle, gathers both; asserts pools and outputs agree."""
    k_pool, v_pool = new_pools(iva, dev, num_pages, hkv, d, bs, dtype, canary)
    iva.kv_append(k_new.to(dev), v_new.to(dev), k_pool, v_pool, slots.to(dev))
    ko, vo = iva.kv_gather(k_pool, v_pool, layout.block_tables.to(dev),
                           layout.context_lens.to(dev), out_len=out_len)
    ok, ov = oracle_pools(num_pages, hkv, d, bs, dtype, canary)
    orc.append(ok, ov, bits(k_new), bits(v_new), slots.numpy())
    ek, ev = orc.gather(ok, ov, layout.block_tables.numpy(), layout.context_lens.numpy(),
                        out_len=out_len)
    assert np.array_equal(bits(k_pool), ok), "K pool differs from oracle"
    assert np.array_equal(bits(v_pool), ov), "V pool differs from oracle"
    assert np.array_equal(bits(ko), ek), "gathered K differs from oracle"
    assert np.array_equal(bits(vo), ev), "gathered V differs from oracle"
    return ko, vo


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_c1_round_trip(iva, dev, dtype):
    w = iva.workloads.c1_append_gather(seed=0, dtype=dtype)
    lay = w["layout"]
    ko, vo = run_case(iva, dev, w["k_new"], w["v_new"], w["slot_mapping"], lay, w["num_pages"],
                      w["num_kv_heads"], w["head_dim"], 16, dtype)
    # round trip: sequence b's gathered rows are exactly its appended rows
    start = 0
    for b, n in enumerate(w["lengths"]):
        rows_k = w["k_new"][start:start + n].transpose(0, 1)  # [Hkv, n, D]
        rows_v = w["v_new"][start:start + n].transpose(0, 1)
        assert np.array_equal(bits(ko[b, :, :n]), bits(rows_k))
        assert np.array_equal(bits(vo[b, :, :n]), bits(rows_v))
        assert not bits(ko[b, :, n:]).any() and not bits(vo[b, :, n:]).any()
        start += n


def test_c1_golden_digest(iva, dev):
    """C1 fp32 outputs match the committed SHA-256 digests (tests/golden/c1.json)."""
    gold = json.loads((GOLDEN / "c1.json").read_text())
    w = iva.workloads.c1_append_gather(seed=gold["seed"])
    assert hashlib.sha256(bits(w["k_new"]).tobytes()).hexdigest() == gold["k_new_sha256"]
    lay = w["layout"]
    k_pool, v_pool = new_pools(iva, dev, w["num_pages"], 8, 64, 16, torch.float32)
    iva.kv_append(w["k_new"].to(dev), w["v_new"].to(dev), k_pool, v_pool, w["slot_mapping"].to(dev))
    ko, vo = iva.kv_gather(k_pool, v_pool, lay.block_tables.to(dev), lay.context_lens.to(dev))
    assert hashlib.sha256(bits(ko).tobytes()).hexdigest() == gold["k_out_sha256"]
    assert hashlib.sha256(bits(vo).tobytes()).hexdigest() == gold["v_out_sha256"]


def test_canary_and_skipped_slots(iva, dev):
    """Slots -1 and out-of-range are skipped; every untouched pool word keeps the canary."""
    w = iva.workloads.c1_append_gather(seed=3, dtype=torch.float16)
    slots = w["slot_mapping"].clone()
    slots[::7] = -1
    slots[5] = w["num_pages"] * 16       # one past the pool
    slots[11] = 2 ** 30                  # far out of range
    run_case(iva, dev, w["k_new"], w["v_new"], slots, w["layout"], w["num_pages"], 8, 64, 16,
             torch.float16, canary=0x7E5A)


def test_empty_inputs(iva, dev):
    k_pool, v_pool = new_pools(iva, dev, 4, 2, 64, 16, torch.float16)
    empty = torch.empty(0, 2, 64, dtype=torch.float16, device=dev)
    iva.kv_append(empty, empty, k_pool, v_pool, torch.empty(0, dtype=torch.int32, device=dev))
    assert not bits(k_pool).any()
    bt = torch.empty(0, 3, dtype=torch.int32, device=dev)
    ko, vo = iva.kv_gather(k_pool, v_pool, bt, torch.empty(0, dtype=torch.int32, device=dev))
    assert ko.shape == (0, 2, 48, 64)
    # zero-length sequences gather to all-zero rows
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=dev)
    k_pool.fill_(1.0)
    ko, vo = iva.kv_gather(k_pool, v_pool, bt, torch.zeros(2, dtype=torch.int32, device=dev))
    assert not bits(ko).any() and not bits(vo).any()


def test_invalid_pages_and_out_len(iva, dev):
    """Invalid page ids read as zero rows; out_len truncates or zero-pads."""
    w = iva.workloads.c1_append_gather(seed=4, dtype=torch.bfloat16)
    lay = w["layout"]
    bt = lay.block_tables.clone()
    bt[1, 2] = -5
    bt[2, 0] = w["num_pages"] + 3
    lay2 = iva.workloads.PagedLayout(lay.lengths, bt, lay.num_pages)
    for out_len in (None, 100, 300, 1):
        run_case(iva, dev, w["k_new"], w["v_new"], w["slot_mapping"], lay2, w["num_pages"], 8, 64,
                 16, torch.bfloat16, out_len=out_len)


def test_context_longer_than_table(iva, dev):
    """context_lens beyond max_blocks * block_size: the missing pages gather as zeros."""
    w = iva.workloads.c1_append_gather(seed=5)
    lay = w["layout"]
    ctx = lay.context_lens.clone()
    ctx[3] = 1000
    lay2 = iva.workloads.PagedLayout(ctx.tolist(), lay.block_tables, lay.num_pages)
    run_case(iva, dev, w["k_new"], w["v_new"], w["slot_mapping"], lay2, w["num_pages"], 8, 64, 16,
             torch.float32, out_len=1024)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_strided_and_misaligned_sources(iva, dev, dtype):
    """K/V as views into a fused [n, 3, Hkv, D] projection (strided) and at a
    misaligned offset (scalar path) append the same bits as contiguous rows."""
    w = iva.workloads.c1_append_gather(seed=6, dtype=dtype)
    n = w["k_new"].shape[0]
    fused = torch.empty(n, 3, 8, 64, dtype=dtype)
    fused[:, 1] = w["k_new"]
    fused[:, 2] = w["v_new"]
    fused = fused.to(dev)
    k_view, v_view = fused[:, 1], fused[:, 2]
    assert not k_view.is_contiguous()
    ref_k, ref_v = new_pools(iva, dev, w["num_pages"], 8, 64, 16, dtype)
    iva.kv_append(w["k_new"].to(dev), w["v_new"].to(dev), ref_k, ref_v, w["slot_mapping"].to(dev))
    k_pool, v_pool = new_pools(iva, dev, w["num_pages"], 8, 64, 16, dtype)
    iva.kv_append(k_view, v_view, k_pool, v_pool, w["slot_mapping"].to(dev))
    assert torch.equal(bits_t(k_pool), bits_t(ref_k)) and torch.equal(bits_t(v_pool), bits_t(ref_v))
    flat = torch.empty(n * 8 * 64 + 1, dtype=dtype, device=dev)
    kmis = flat[1:].view(n, 8, 64)
    kmis.copy_(w["k_new"].to(dev))
    k_pool.zero_(), v_pool.zero_()
    iva.kv_append(kmis, w["v_new"].to(dev), k_pool, v_pool, w["slot_mapping"].to(dev))
    assert torch.equal(bits_t(k_pool), bits_t(ref_k)) and torch.equal(bits_t(v_pool), bits_t(ref_v))


def bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.view(BITS[t.dtype][0])


@pytest.mark.parametrize("dtype,d,bs", [(torch.float16, 8, 16), (torch.float16, 128, 16),
                                        (torch.float16, 256, 16), (torch.bfloat16, 64, 16),
                                        (torch.float32, 4, 8),
                                        (torch.bfloat16, 64, 32), (torch.float32, 128, 1),
                                        (torch.float16, 72, 5)])
def test_geometries(iva, dev, dtype, d, bs):
    lengths = [1, bs - 1 if bs > 1 else 1, bs, 3 * bs + 2]
    hkv = 5  # the gather's workgroups take four kv heads: a full group and a partial one
    gen = torch.Generator().manual_seed(d * 31 + bs)
    need = sum(-(-n // bs) for n in lengths)
    lay = iva.workloads.permuted_layout(lengths, need + 5, gen, block_size=bs)
    n_tok = sum(lengths)
    k_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    v_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    slots = torch.cat([lay.slots(b, torch.arange(n)) for b, n in enumerate(lengths)])
    run_case(iva, dev, k_new, v_new, slots, lay, need + 5, hkv, d, bs, dtype, canary=0x1234)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize("rows", [32, 4080, 4096], ids=lambda n: f"{n}rows")
def test_launch_shapes_around_the_few_row_switch(iva, dev, dtype, rows):
    """The appends take one kv head per lane below 1024 waves of eight heads per lane
    (fp16, 8 kv heads, head_dim 128: below 4096 rows) and eight heads per lane above; a
    decode step's rows (32 sequences, one row each, at random rows of their pages) and
    chunk appends on both sides of the switch are bit-exact, plain and with RoPE (the
    RoPE form against rope_ followed by the plain append)."""
    gen = torch.Generator().manual_seed(rows)
    hkv, d = 8, 128
    if rows == 32:
        lengths = [int(x) for x in torch.randint(1, 300, (32,), generator=gen)]
    else:
        lengths = [rows // 2 + 5, rows - rows // 2 - 5]
    need = sum(-(-n // 16) for n in lengths)
    lay = iva.workloads.permuted_layout(lengths, need + 3, gen)
    if rows == 32:  # the last position of each sequence: one row per page
        slots = torch.cat([lay.slots(b, torch.tensor([n - 1])) for b, n in enumerate(lengths)])
    else:
        slots = torch.cat([lay.slots(b, torch.arange(n)) for b, n in enumerate(lengths)])
    n_tok = slots.numel()
    k_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    v_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    k_pool, v_pool = new_pools(iva, dev, need + 3, hkv, d, 16, dtype, 0x1234)
    iva.kv_append(k_new.to(dev), v_new.to(dev), k_pool, v_pool, slots.to(dev))
    ok, ov = oracle_pools(need + 3, hkv, d, 16, dtype, 0x1234)
    orc.append(ok, ov, bits(k_new), bits(v_new), slots.numpy())
    assert np.array_equal(bits(k_pool), ok) and np.array_equal(bits(v_pool), ov)
    pos = torch.randint(0, 1 << 15, (n_tok,), generator=gen).to(torch.int32).to(dev)
    out = []
    for fused in (True, False):
        kp, vp = new_pools(iva, dev, need + 3, hkv, d, 16, dtype, 0x1234)
        if fused:
            iva.kv_append(k_new.to(dev), v_new.to(dev), kp, vp, slots.to(dev), rope_positions=pos)
        else:
            iva.kv_append(iva.rope_(k_new.to(dev).clone(), pos), v_new.to(dev), kp, vp, slots.to(dev))
        out.append((bits(kp), bits(vp)))
    assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1])


def test_decode_appends_and_prefill_chunk(iva, dev):
    """C5-style traffic: one 512-token prefill chunk and one-token decode appends for 32
    sequences, interleaved, on a fp16 Hkv 8 / D 128 pool."""
    gen = torch.Generator().manual_seed(9)
    lengths = [int(x) for x in torch.randint(1, 900, (32,), generator=gen)]
    lengths[0] = 512 + 33
    lay = iva.workloads.permuted_layout([n + 1 for n in lengths], 2200, gen)
    d, hkv = 128, 8
    rows_k = [torch.randn(n + 1, hkv, d, generator=gen).half() for n in lengths]
    rows_v = [torch.randn(n + 1, hkv, d, generator=gen).half() for n in lengths]
    k_pool, v_pool = new_pools(iva, dev, 2200, hkv, d, 16, torch.float16)
    ok, ov = oracle_pools(2200, hkv, d, 16, torch.float16)
    # prefill: every sequence's first n rows (one big append)
    kk = torch.cat([r[:n] for r, n in zip(rows_k, lengths)])
    vv = torch.cat([r[:n] for r, n in zip(rows_v, lengths)])
    slots = torch.cat([lay.slots(b, torch.arange(n)) for b, n in enumerate(lengths)])
    iva.kv_append(kk.to(dev), vv.to(dev), k_pool, v_pool, slots.to(dev))
    orc.append(ok, ov, bits(kk), bits(vv), slots.numpy())
    # decode step: one row per sequence at position n
    kk = torch.stack([r[n] for r, n in zip(rows_k, lengths)])
    vv = torch.stack([r[n] for r, n in zip(rows_v, lengths)])
    slots = torch.stack([lay.slots(b, torch.tensor(n)) for b, n in enumerate(lengths)])
    iva.kv_append(kk.to(dev), vv.to(dev), k_pool, v_pool, slots.to(dev))
    orc.append(ok, ov, bits(kk), bits(vv), slots.numpy())
    assert np.array_equal(bits(k_pool), ok) and np.array_equal(bits(v_pool), ov)
    ko, vo = iva.kv_gather(k_pool, v_pool, lay.block_tables.to(dev), lay.context_lens.to(dev))
    for b, n in enumerate(lengths):
        assert np.array_equal(bits(ko[b, :, :n + 1]), bits(rows_k[b].transpose(0, 1)))
        assert np.array_equal(bits(vo[b, :, :n + 1]), bits(rows_v[b].transpose(0, 1)))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
def test_chunks_starting_mid_page(iva, dev, dtype):
    """Chunked prefill after decode steps: every sequence already holds L_b rows (most not
    a multiple of 16), and one call appends a 512-row chunk to each of 10 sequences, so
    every chunk starts mid-page and neighbouring token groups share pages.  Pools
    bit-identical to the oracle's; with RoPE fused, bit-identical to rope_ followed by
    the plain append of the rotated rows."""
    gen = torch.Generator().manual_seed(21)
    prior = [int(x) for x in torch.randint(1, 900, (10,), generator=gen)]
    prior[0], prior[1] = 16 * 7, 16 * 3 + 15    # one aligned start, one a row before a page
    chunk, hkv, d = 512, 8, 128
    total = [n + chunk for n in prior]
    num_pages = sum(-(-n // 16) for n in total) + 5
    lay = iva.workloads.permuted_layout(total, num_pages, gen)
    n_tok = 10 * chunk
    k_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    v_new = torch.randn(n_tok, hkv, d, generator=gen).to(dtype)
    slots = torch.cat([lay.slots(b, torch.arange(n, n + chunk)) for b, n in enumerate(prior)])
    assert sum(n % 16 != 0 for n in prior) >= 8
    k_pool, v_pool = new_pools(iva, dev, num_pages, hkv, d, 16, dtype, canary=0x1234)
    iva.kv_append(k_new.to(dev), v_new.to(dev), k_pool, v_pool, slots.to(dev))
    ok, ov = oracle_pools(num_pages, hkv, d, 16, dtype, canary=0x1234)
    orc.append(ok, ov, bits(k_new), bits(v_new), slots.numpy())
    assert np.array_equal(bits(k_pool), ok) and np.array_equal(bits(v_pool), ov)
    if dtype == torch.float32:
        return
    pos = torch.cat([torch.arange(n, n + chunk) for n in prior]).to(torch.int32).to(dev)
    kf, vf = new_pools(iva, dev, num_pages, hkv, d, 16, dtype, canary=0x1234)
    iva.kv_append(k_new.to(dev), v_new.to(dev), kf, vf, slots.to(dev), rope_positions=pos)
    kr, vr = new_pools(iva, dev, num_pages, hkv, d, 16, dtype, canary=0x1234)
    k_rot = iva.rope_(k_new.to(dev).clone(), pos)
    iva.kv_append(k_rot, v_new.to(dev), kr, vr, slots.to(dev))
    assert torch.equal(bits_t(kf), bits_t(kr)) and torch.equal(bits_t(vf), bits_t(vr))


def bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.view(BITS[t.dtype][0])


def test_argument_errors(iva, dev):
    k_pool, v_pool = new_pools(iva, dev, 4, 2, 64, 16, torch.float16)
    rows = torch.zeros(3, 2, 64, dtype=torch.float16, device=dev)
    with pytest.raises(TypeError):
        iva.kv_append(rows.float(), rows.float(), k_pool, v_pool,
                      torch.zeros(3, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        iva.kv_append(rows, rows, k_pool, v_pool, torch.zeros(2, dtype=torch.int32, device=dev))
    with pytest.raises(TypeError):
        iva.kv_append(rows, rows, k_pool, v_pool, torch.zeros(3, dtype=torch.int64, device=dev))
    with pytest.raises(RuntimeError):
        iva.kv_append(rows.cpu(), rows.cpu(), k_pool, v_pool,
                      torch.zeros(3, dtype=torch.int32, device=dev))
