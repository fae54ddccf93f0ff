"""Seeded random shapes through every decode and prefill path, against the fp64 oracle.

Each case draws a batch size, kv heads, GQA group, head_dim, dtype, ragged context
lengths (empty sequences and page boundaries included), a sliding window and sinks,
then checks the stream walk, the partitioned walk, the fused append + attend op (pools
bit-identical to ivakv_append of the same rows; it takes the stream walk or, for
batches with a unit per CU and short tables, one partition per sequence) and chunked
prefill, single-launch and split.  Tolerance as in the other GPU tests: 2e-3 (fp16 / bf16) or 1e-5 (fp32) plus
one half-ulp of the output dtype times the exact value.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

ATOL = {torch.float16: 2e-3, torch.bfloat16: 2e-3, torch.float32: 1e-5}
OUT_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}
DTYPES = [torch.float16, torch.bfloat16, torch.float32]


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_close(out, ref, dtype, what):
    err = np.abs(to_np(out) - ref)
    bound = ATOL[dtype] + OUT_ULP[dtype] * np.abs(ref)
    assert (err <= bound).all(), f"{what}: max abs err {err.max():.3e}"


def draw(seed: int):
    rng = np.random.default_rng(seed)
    big = seed % 4 == 0  # every fourth case: one to four units per CU, so decode runs one partition
    hkv = int(rng.choice([4, 8])) if big else int(rng.choice([1, 2, 4, 8]))
    batch = (256 // hkv + int(rng.integers(0, 8))) if big else int(rng.integers(1, 40))
    g = int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128, 256]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    hi = 900 if big else 1500
    lengths = rng.integers(0, hi, batch).tolist()
    for i, special in enumerate((0, 1, 16, 17)[: batch // 4]):
        lengths[i] = special
    window, n_sink = 0, 0
    if rng.random() < 0.4:
        window = int(rng.integers(1, 400))
        n_sink = int(rng.integers(0, 6))
    return batch, hkv, g, d, dtype, lengths, window, n_sink


@pytest.mark.parametrize("seed", range(16))
def test_decode_paths_random(iva, dev, seed):
    batch, hkv, g, d, dtype, lengths, window, n_sink = draw(seed)
    what = f"seed {seed}: B={batch} Hkv={hkv} G={g} D={d} {dtype} w={window} s={n_sink}"
    base = iva.workloads.decode_batch(lengths, hkv * g, hkv, d, dtype, seed=200 + seed,
                                      scale=d ** -0.5, extra_pages=2)
    lay = base["layout"]
    q, kp, vp = base["q"].to(dev), base["k_pool"].to(dev), base["v_pool"].to(dev)
    bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
    ref = orc.decode_attention(to_np(base["q"]), to_np(base["k_pool"]), to_np(base["v_pool"]),
                               lay.block_tables.numpy(), lay.context_lens.numpy(),
                               window=window, n_sink=n_sink)
    # default walk: the stream walk, or one partition per sequence in a single launch for
    # one to four units per CU on short tables (every fourth seed)
    assert_close(iva.paged_decode_attention(q, kp, vp, bt, ctx, window=window, n_sink=n_sink),
                 ref, dtype, "default " + what)
    assert_close(iva.paged_decode_attention(q, kp, vp, bt, ctx, window=window, n_sink=n_sink,
                                            partition_pages=8), ref, dtype, "partitioned " + what)

    # fused append + attend: the new token of sequence b sits at position L_b - 1
    gen = torch.Generator().manual_seed(300 + seed)
    k_new = (torch.randn(batch, hkv, d, generator=gen) * d ** -0.5).to(dtype)
    v_new = (torch.randn(batch, hkv, d, generator=gen) * d ** -0.5).to(dtype)
    tb = lay.block_tables
    slots = torch.tensor([int(tb[b, (n - 1) // 16]) * 16 + (n - 1) % 16 if n > 0 else -1
                          for b, n in enumerate(lengths)], dtype=torch.int32)
    kp_a, vp_a = kp.clone(), vp.clone()
    iva.kv_append(k_new.to(dev), v_new.to(dev), kp_a, vp_a, slots.to(dev))
    kp_f, vp_f = kp.clone(), vp.clone()
    out = iva.paged_decode_append_attention(q, k_new.to(dev), v_new.to(dev), kp_f, vp_f, bt, ctx,
                                            window=window, n_sink=n_sink)
    ti = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(kp_a.view(ti), kp_f.view(ti)) and torch.equal(vp_a.view(ti), vp_f.view(ti)), what
    ref_f = orc.decode_attention(to_np(base["q"]), to_np(kp_a), to_np(vp_a),
                                 lay.block_tables.numpy(), lay.context_lens.numpy(),
                                 window=window, n_sink=n_sink)
    assert_close(out, ref_f, dtype, "fused " + what)


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random(iva, dev, seed):
    batch, hkv, g, d, dtype, lengths, window, n_sink = draw(1000 + seed)
    batch = min(batch, 12)
    lengths = [max(n, 1) for n in lengths[:batch]]
    rng = np.random.default_rng(seed)
    chunks = [int(rng.integers(0, n + 1)) for n in lengths]
    what = f"seed {seed}: B={batch} Hkv={hkv} G={g} D={d} {dtype} w={window} s={n_sink}"
    c = iva.workloads.prefill_batch(lengths, chunks, hkv * g, hkv, d, dtype, seed=400 + seed,
                                    scale=d ** -0.5)
    lay = c["layout"]
    ref = orc.prefill_attention(to_np(c["q"]), to_np(c["k_pool"]), to_np(c["v_pool"]),
                                lay.block_tables.numpy(), lay.context_lens.numpy(),
                                c["query_start"].numpy(), window=window, n_sink=n_sink)
    # the single-launch kernel and the split path (segments of >= 16 pairs: contexts
    # past 512 keys split)
    for split in (False, True):
        out = iva.paged_prefill_attention(c["q"].to(dev), c["k_pool"].to(dev),
                                          c["v_pool"].to(dev), lay.block_tables.to(dev),
                                          lay.context_lens.to(dev), c["query_start"].to(dev),
                                          window=window, n_sink=n_sink, split=split)
        assert_close(out, ref, dtype, f"prefill split={split} " + what)
