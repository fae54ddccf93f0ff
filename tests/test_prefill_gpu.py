"""Paged prefill / chunked-prefill attention on the GPU vs the fp64 CPU oracle.

Tolerance (north star): max |out - exact| <= 2e-3 for fp16/bf16 and 1e-5 for fp32,
plus one half-ulp of the output dtype times |exact| (output rounding), as for decode.
Cases cover full prefill (chunk = whole sequence), chunks after a cached prefix,
single-row chunks, empty chunks, chunks longer than the context (rows at negative
positions are zero), invalid page ids, NaN bits past the context, GQA groups 1, 3, 4
and 8, windows with sinks, and head_dim 64 / 128 / 256.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

ATOL = {torch.float16: 2e-3, torch.bfloat16: 2e-3, torch.float32: 1e-5}
OUT_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_close(out, ref, dtype, what=""):
    err = np.abs(to_np(out) - ref)
    bound = ATOL[dtype] + OUT_ULP[dtype] * np.abs(ref)
    worst = float((err - bound).max()) if err.size else -1.0
    assert worst <= 0.0, f"{what}: max abs err {err.max():.3e} exceeds bound (excess {worst:.3e})"


def make(iva, lengths, chunks, hq, hkv, d, dtype, seed=0):
    return iva.workloads.prefill_batch(lengths, chunks, hq, hkv, d, dtype, seed=seed,
                                       scale=d ** -0.5)


def oracle(c, bt=None, window=0, n_sink=0):
    lay = c["layout"]
    return orc.prefill_attention(to_np(c["q"]), to_np(c["k_pool"]), to_np(c["v_pool"]),
                                 (lay.block_tables if bt is None else bt).numpy(),
                                 lay.context_lens.numpy(), c["query_start"].numpy(),
                                 window=window, n_sink=n_sink)


def run(iva, dev, c, bt=None, **kw):
    lay = c["layout"]
    return iva.paged_prefill_attention(c["q"].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev),
                                       (lay.block_tables if bt is None else bt).to(dev),
                                       lay.context_lens.to(dev), c["query_start"].to(dev), **kw)


CASES = {
    "full": ([16, 100], [16, 100]),
    "chunk_after_prefix": ([257, 70, 33], [64, 70, 1]),
    "ragged": ([1, 17, 300, 45], [1, 17, 37, 0]),
    "longer_than_context": ([5, 40], [9, 40]),
}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("heads", [(8, 2), (4, 4), (12, 4), (16, 2)], ids=lambda h: f"{h[0]}q{h[1]}kv")
def test_prefill_vs_oracle(iva, dev, dtype, case, heads):
    lengths, chunks = CASES[case]
    c = make(iva, lengths, chunks, heads[0], heads[1], 64, dtype, seed=3)
    out = run(iva, dev, c)
    assert_close(out, oracle(c), dtype, f"{case} {heads} {dtype}")


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("window,sink", [(0, 0), (50, 4), (16, 0), (1, 1)])
def test_prefill_head_dims_windows(iva, dev, d, dtype, window, sink):
    c = make(iva, [190, 77], [120, 77], 8, 2, d, dtype, seed=5)
    out = run(iva, dev, c, window=window, n_sink=sink)
    assert_close(out, oracle(c, window=window, n_sink=sink), dtype, f"D={d} w={window} s={sink}")


def test_prefill_invalid_pages_and_nan_tail(iva, dev):
    """Keys on an invalid page id are not attended; NaN bits past the context (the
    tail of the last page) never reach the output."""
    c = make(iva, [70, 41], [30, 41], 8, 2, 128, torch.float16, seed=7)
    bt = c["layout"].block_tables.clone()
    bt[0, 1] = -1
    bt[1, 0] = c["layout"].num_pages + 5
    last = int(c["layout"].block_tables[1, 2])  # length 41: rows 9..15 of page 2 are past it
    c["k_pool"][last, :, :, 9:] = float("nan")
    c["v_pool"][last, :, :, 9:] = float("nan")
    out = run(iva, dev, c, bt=bt, window=24, n_sink=2)
    assert torch.isfinite(out).all()
    assert_close(out, oracle(c, bt=bt, window=24, n_sink=2), torch.float16, "invalid pages")


@pytest.mark.parametrize("dtype,d", [(torch.float16, 128), (torch.bfloat16, 128),
                                     (torch.float32, 128), (torch.float16, 256)], ids=str)
@pytest.mark.parametrize("chunked", [False, True], ids=["full", "chunk33"])
def test_prefill_walk_lengths_and_mid_walk_holes(iva, dev, dtype, d, chunked):
    """Causal walks of 1 to 8 page pairs (the pipelined loop loads past the last pair;
    odd and even pair counts) with an invalid page id and an out-of-range one in the
    middle of the longer walks, NaN bits on the pages those ids replaced and past every
    context: pairs holding a hole or the context's end take masks, the rest none.
    fp32 and head_dim 256 run the unpipelined loop."""
    lengths = [15, 16, 17, 32, 33, 64, 65, 96, 97, 128, 160, 161, 224, 250]
    chunks = [min(n, 33) for n in lengths] if chunked else lengths
    c = make(iva, lengths, chunks, 8, 2, d, dtype, seed=13)
    lay = c["layout"]
    bt = lay.block_tables.clone()
    for b, n in enumerate(lengths):
        if n % 16:  # the tail of the last page
            last = int(lay.block_tables[b, (n - 1) // 16])
            c["k_pool"][last, :, :, n % 16:] = float("nan")
            c["v_pool"][last, :, :, n % 16:] = float("nan")
        if n >= 128:  # holes in the middle of the walk; the replaced pages hold NaN
            for j, bad in ((3, -1), (6, lay.num_pages + 3)):
                c["k_pool"][int(bt[b, j])] = float("nan")
                c["v_pool"][int(bt[b, j])] = float("nan")
                bt[b, j] = bad
    out = run(iva, dev, c, bt=bt)
    assert torch.isfinite(out).all()
    assert_close(out, oracle(c, bt=bt), dtype, "walk lengths / holes")


def test_chunked_equals_full_and_last_row_equals_decode(iva, dev):
    """Prefill in three chunks == one full prefill (both vs the oracle), and the last
    row equals the decode kernel's output for that position."""
    length, hq, hkv, d = 300, 8, 2, 128
    c = make(iva, [length], [length], hq, hkv, d, torch.bfloat16, seed=9)
    full = run(iva, dev, c, window=100, n_sink=4)
    parts = []
    for lo, hi in ((0, 45), (45, 200), (200, 300)):
        cc = dict(c, q=c["q"][lo:hi], query_start=torch.tensor([0, hi - lo], dtype=torch.int32))
        cc["layout"] = type(c["layout"])([hi], c["layout"].block_tables, c["layout"].num_pages)
        parts.append(run(iva, dev, cc, window=100, n_sink=4))
    chunked = torch.cat(parts)
    ref = oracle(c, window=100, n_sink=4)
    assert_close(full, ref, torch.bfloat16, "full")
    assert_close(chunked, ref, torch.bfloat16, "chunked")
    dec = iva.paged_decode_attention(c["q"][-1:].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev),
                                     c["layout"].block_tables.to(dev),
                                     c["layout"].context_lens.to(dev), window=100, n_sink=4)
    assert (full[-1].float() - dec[0].float()).abs().max().item() <= 2e-3


def test_prefill_c5_chunk_size(iva, dev):
    """A 512-token chunk on top of a 1536-token prefix, 4 sequences, GQA 32/8, D 128, fp16."""
    c = make(iva, [2048, 1700, 900, 512], [512, 512, 512, 512], 32, 8, 128, torch.float16, seed=11)
    out = run(iva, dev, c)
    ref = oracle(c)
    err = np.abs(to_np(out) - ref).max()
    assert err <= 2e-3, err


def test_prefill_argument_errors(iva, dev):
    c = make(iva, [20], [20], 4, 2, 64, torch.float16)
    lay = c["layout"]
    args = (c["q"].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev), lay.block_tables.to(dev),
            lay.context_lens.to(dev))
    with pytest.raises(TypeError, match="query_start"):
        iva.paged_prefill_attention(*args, c["query_start"].to(dev).long())
    with pytest.raises(ValueError, match="B\\+1"):
        iva.paged_prefill_attention(*args, c["query_start"][:1].to(dev))
    with pytest.raises(TypeError, match="dtype"):
        iva.paged_prefill_attention(args[0].float(), *args[1:], c["query_start"].to(dev))
    out = iva.paged_prefill_attention(*args, c["query_start"].to(dev), max_query_len=0)
    assert out.shape == c["q"].shape  # nothing computed, no error
    # query_start must rise from 0 to n_tok (checked when max_query_len is read from it)
    for qs in ([1, 20], [0, 19], [0, 21]):
        with pytest.raises(ValueError, match="query_start"):
            iva.paged_prefill_attention(*args, torch.tensor(qs, dtype=torch.int32, device=dev))


def test_prefill_skips_sequences_outside_q(iva, dev):
    """With max_query_len given there is no host read of query_start: the kernel skips
    a sequence whose rows [query_start[b], query_start[b+1]) do not lie inside q (its
    output rows stay as they were) and computes the others."""
    c = make(iva, [40, 30, 25], [8, 6, 5], 4, 2, 64, torch.float16, seed=3)
    lay = c["layout"]
    n_tok = c["q"].shape[0]          # 19 rows: 0..7, 8..13, 14..18
    want = run(iva, dev, c)
    qs = torch.tensor([0, 8, 14, 21], dtype=torch.int32, device=dev)   # last ends past q
    out = torch.full_like(want, 7.0)
    iva.paged_prefill_attention(c["q"].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev),
                                lay.block_tables.to(dev), lay.context_lens.to(dev), qs,
                                max_query_len=8, out=out)
    assert torch.equal(out[:14], want[:14])
    assert bool((out[14:] == 7.0).all())
    qs = torch.tensor([-3, 8, 14, n_tok], dtype=torch.int32, device=dev)  # first before q
    out = torch.full_like(want, 7.0)
    iva.paged_prefill_attention(c["q"].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev),
                                lay.block_tables.to(dev), lay.context_lens.to(dev), qs,
                                max_query_len=11, out=out)
    assert bool((out[:8] == 7.0).all())
    assert torch.equal(out[8:], want[8:])


@pytest.mark.parametrize("scale", [-0.2, 0.0, 0.35])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=str)
def test_prefill_explicit_scales(iva, dev, scale, dtype):
    """Non-default scales, including negative (the kernel negates q) and zero (uniform
    weights over the visible keys)."""
    c = make(iva, [90, 33], [40, 33], 8, 2, 64, dtype, seed=13)
    lay = c["layout"]
    out = run(iva, dev, c, scale=scale, window=20, n_sink=2)
    ref = orc.prefill_attention(to_np(c["q"]), to_np(c["k_pool"]), to_np(c["v_pool"]),
                                lay.block_tables.numpy(), lay.context_lens.numpy(),
                                c["query_start"].numpy(), scale=scale, window=20, n_sink=2)
    assert_close(out, ref, dtype, f"scale {scale}")
