"""Split prefill (ivakv_prefill_attn_split): every row block's walk cut along the keys into
segments, run on a persistent grid from per-XCD queues and merged by log-sum-exp,
against the fp64 CPU oracle with the bounds of tests/test_prefill_gpu.py (2e-3 for
fp16 / bf16, 1e-5 for fp32, plus half an output ulp of |exact|).

Segments are at least 16 pairs (512 keys), and the plan sizes them to the batch's
work per CU, so these cases put chunks on contexts of 600 - 9000 keys to split row
blocks into 2 - 16 segments; cases with short contexts run the same grid unsplit.
The plan's own invariants are read back from the workspace: every queue ticket is
taken exactly once, and the split row blocks fit the 512 partial slots.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

ATOL = {torch.float16: 2e-3, torch.bfloat16: 2e-3, torch.float32: 1e-5}
OUT_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}
SLOTS = 512


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


def dev_args(c, dev, bt=None):
    lay = c["layout"]
    return (c["q"].to(dev), c["k_pool"].to(dev), c["v_pool"].to(dev),
            (lay.block_tables if bt is None else bt).to(dev), lay.context_lens.to(dev),
            c["query_start"].to(dev))


def run(iva, dev, c, bt=None, **kw):
    return iva.paged_prefill_attention(*dev_args(c, dev, bt), **kw)


def grid_wgs(dev) -> int:
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    return cus & ~7 if cus >= 16 else 8


SPLIT_CASES = {
    # (context lengths, chunk lengths)
    "one_long_chunk": ([4000], [64]),
    "chunks_after_prefixes": ([2000, 700, 1100, 90], [64, 70, 1, 90]),
    "mixed_with_empty": ([3000, 17, 1500, 600], [200, 17, 0, 33]),
    "full_prefill_long": ([1200], [1200]),
}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("case", list(SPLIT_CASES))
@pytest.mark.parametrize("heads", [(8, 2), (4, 4), (12, 4)], ids=lambda h: f"{h[0]}q{h[1]}kv")
def test_split_vs_oracle(iva, dev, dtype, case, heads):
    lengths, chunks = SPLIT_CASES[case]
    c = make(iva, lengths, chunks, heads[0], heads[1], 64, dtype, seed=21)
    out = run(iva, dev, c, split=True)
    assert_close(out, oracle(c), dtype, f"{case} {heads} {dtype}")


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("window,sink", [(0, 0), (700, 4), (100, 0)])
def test_split_head_dims_windows(iva, dev, d, dtype, window, sink):
    c = make(iva, [2600, 1000], [40, 300], 8, 2, d, dtype, seed=23)
    out = run(iva, dev, c, split=True, window=window, n_sink=sink)
    assert_close(out, oracle(c, window=window, n_sink=sink), dtype, f"D{d} w{window} s{sink}")


def test_split_holes_and_nan_tails(iva, dev):
    """Invalid and out-of-range page ids inside split walks (NaN on the pages they
    replaced) and NaN bits past every context: masked in every segment."""
    lengths, chunks = [2500, 1900, 777], [100, 33, 20]
    c = make(iva, lengths, chunks, 8, 2, 128, torch.float16, seed=29)
    lay = c["layout"]
    bt = lay.block_tables.clone()
    for b, n in enumerate(lengths):
        if n % 16:
            last = int(lay.block_tables[b, (n - 1) // 16])
            c["k_pool"][last, :, :, n % 16:] = float("nan")
            c["v_pool"][last, :, :, n % 16:] = float("nan")
        for j, bad in ((5, -1), (40, lay.num_pages + 3)):
            if j < (n - 1) // 16:
                c["k_pool"][int(bt[b, j])] = float("nan")
                c["v_pool"][int(bt[b, j])] = float("nan")
                bt[b, j] = bad
    out = run(iva, dev, c, bt=bt, split=True)
    assert torch.isfinite(out).all()
    assert_close(out, oracle(c, bt=bt), torch.float16, "holes")


def test_split_equals_unsplit_and_c5_chunks(iva, dev):
    """A 512-token chunk on each of four prefixes (C5's chunk size, GQA 32/8, D 128,
    fp16): the split and the single-launch kernels both within the bound of the exact
    output (the two differ only by where P is rounded against which running max)."""
    c = make(iva, [5000, 2048, 900, 512], [512, 512, 512, 512], 32, 8, 128, torch.float16,
             seed=11)
    ref = oracle(c)
    split = run(iva, dev, c, split=True)
    plain = run(iva, dev, c, split=False)
    assert_close(split, ref, torch.float16, "split")
    assert_close(plain, ref, torch.float16, "plain")


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("window,sink", [(0, 0), (500, 4)])
def test_split_fp8_pages(iva, dev, qdt, window, sink):
    """FP8 pools (garbage codes past every context) through the split path, against
    the fp64 oracle's prefill over the dequantized pages, as tests/test_fp8_gpu.py
    checks the single-launch kernel."""
    from test_fp8_gpu import append_both, fp8_case
    lengths, chunks = [3000, 1400, 45], [64, 200, 45]
    hq, hkv, d = 8, 2, 128
    c = fp8_case(iva, lengths, hkv, d, torch.float32, seed=43, decades=0)
    g, o = append_both(iva, dev, c)
    lay = c["layout"]
    qs = torch.tensor(np.cumsum([0] + chunks), dtype=torch.int32)
    q = (torch.randn(int(qs[-1]), hq, d, generator=torch.Generator().manual_seed(5)) * d ** -0.5).to(qdt)
    out = iva.paged_prefill_attention(q.to(dev), g["k_pool"], g["v_pool"], lay.block_tables.to(dev),
                                      lay.context_lens.to(dev), qs.to(dev), window=window,
                                      n_sink=sink, k_scale=g["k_scale"], v_scale=g["v_scale"],
                                      split=True)
    kd, vd = orc.dequantize_pools(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"], np.float64)
    ref = orc.prefill_attention(q.double().numpy(), kd, vd, lay.block_tables.numpy(),
                                lay.context_lens.numpy(), qs.numpy(), window=window, n_sink=sink)
    assert_close(out, ref, qdt, "fp8 split")


def test_split_plan_invariants_and_garbage_workspace(iva, dev):
    """The plan's counters after a call: queue x holds its virtual units' tickets
    (units x, x + 8, .. times blocks_x) plus one failing grab per workgroup of the
    queue, so every item was taken exactly once and every workgroup left.  The
    workspace starts as random bytes (it needs no initialisation), and two calls in a
    row on it give identical output."""
    lengths, chunks = [4000, 2000, 300], [300, 64, 300]
    hq, hkv, d = 8, 2, 128
    c = make(iva, lengths, chunks, hq, hkv, d, torch.float16, seed=37)
    max_q = max(chunks)
    nbytes = iva.prefill_split_workspace_bytes(len(lengths), hq, hkv, d, max_q, torch.float16)
    ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    out1 = run(iva, dev, c, split=True, workspace=ws, max_query_len=max_q)
    ctl = ws[:256].view(torch.int32).cpu()
    V, n_split, seg = int(ctl[0]), int(ctl[1]), int(ctl[2])
    blocks_x = -(-max_q * (hq // hkv) // 256)
    n_wg = grid_wgs(dev)
    for x in range(8):
        units = (V - x + 7) // 8 if V > x else 0
        assert int(ctl[32 + 4 * x]) == units * blocks_x + n_wg // 8, x
    assert seg >= 16 and seg % 2 == 0
    assert n_split >= 1  # the 4000-key chunk splits
    # every segment of a split block counted in once: the arrival counters (the part
    # after the control block, the unit list and the row-block table) sum to the slots
    up = lambda v: (v + 255) & ~255
    arrive = up(up(up(256) + (len(lengths) * hkv + SLOTS) * 8) + len(lengths) * blocks_x * 8)
    counts = ws[arrive:arrive + 4 * SLOTS].view(torch.int32).cpu()
    assert int(counts.sum()) == int(ctl[3]) > 0
    assert_close(out1, oracle(c), torch.float16, "garbage workspace")
    out2 = run(iva, dev, c, split=True, workspace=ws, max_query_len=max_q)
    assert torch.equal(out1, out2)


def _check_plan(ws, batch, hkv, blocks_x, n_wg):
    """Queue counters: every ticket taken once plus one failing grab per workgroup;
    arrival counters: every split segment counted in once."""
    ctl = ws[:256].view(torch.int32).cpu()
    V = int(ctl[0])
    for x in range(8):
        units = (V - x + 7) // 8 if V > x else 0
        assert int(ctl[32 + 4 * x]) == units * blocks_x + n_wg // 8, x
    up = lambda v: (v + 255) & ~255
    arrive = up(up(up(256) + (batch * hkv + SLOTS) * 8) + batch * blocks_x * 8)
    counts = ws[arrive:arrive + 4 * SLOTS].view(torch.int32).cpu()
    assert int(counts.sum()) == int(ctl[3]) > 0
    return ctl


@pytest.mark.parametrize("batch", [300, 2048])
def test_split_large_batches(iva, dev, batch):
    """Batches past the plan's ranking (more than 256 sequences keep their order) and,
    at 2048 sequences with a 300-token chunk (five row blocks per unit), past the
    row-block table the plan keeps in LDS (more than 8192 blocks: kept in the
    workspace).  Short chunks on short contexts, with two long contexts that split;
    against the fp64 oracle, plan invariants read back.  Batch 2049 is refused."""
    gen = torch.Generator().manual_seed(batch)
    lengths = torch.randint(8, 120, (batch,), generator=gen).tolist()
    chunks = [int(torch.randint(1, min(n, 4) + 1, (1,), generator=gen)) for n in lengths]
    lengths[7], chunks[7] = 5000, 64
    lengths[batch - 50], chunks[batch - 50] = 3000, 300
    hq, hkv, d = 8, 2, 64
    c = make(iva, lengths, chunks, hq, hkv, d, torch.float16, seed=batch % 89)
    max_q = max(chunks)
    nbytes = iva.prefill_split_workspace_bytes(batch, hq, hkv, d, max_q, torch.float16)
    ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    out = run(iva, dev, c, split=True, workspace=ws, max_query_len=max_q)
    blocks_x = -(-max_q * (hq // hkv) // 256)
    assert batch * blocks_x > 8192 or batch == 300
    ctl = _check_plan(ws, batch, hkv, blocks_x, grid_wgs(dev))
    assert int(ctl[1]) >= 2  # both long chunks split
    assert_close(out, oracle(c), torch.float16, f"batch {batch}")
    if batch == 2048:
        c2 = make(iva, lengths + [40], chunks + [2], hq, hkv, d, torch.float16, seed=3)
        with pytest.raises(iva._abi.IvakvError, match="2048"):
            run(iva, dev, c2, split=True)


def test_split_in_a_hip_graph(iva, dev):
    """The three launches captured in one HIP graph (the plan resets the queue
    counters on the device, no host read): every replay, with eager work and
    synchronisations between them, equals the eager result."""
    c = make(iva, [3000, 800], [128, 64], 8, 2, 64, torch.bfloat16, seed=41)
    args = dev_args(c, dev)
    eager = iva.paged_prefill_attention(*args, split=True, max_query_len=128)
    out = torch.empty_like(eager)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        iva.paged_prefill_attention(*args, split=True, max_query_len=128, out=out)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            iva.paged_prefill_attention(*args, split=True, max_query_len=128, out=out)
    torch.cuda.current_stream(dev).wait_stream(stream)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, eager)
        run(iva, dev, c, split=False)  # eager work between replays
        torch.cuda.synchronize(dev)


def test_split_argument_errors(iva, dev):
    c = make(iva, [900], [40], 4, 2, 64, torch.float16)
    args = dev_args(c, dev)
    nbytes = iva.prefill_split_workspace_bytes(1, 4, 2, 64, 40, torch.float16)
    with pytest.raises(ValueError, match="workspace"):
        iva.paged_prefill_attention(*args, split=True,
                                    workspace=torch.empty(nbytes - 1, dtype=torch.uint8, device=dev))
    with pytest.raises(iva._abi.IvakvError, match="workspace"):
        iva._abi.call("ivakv_prefill_attn_split", args[0].data_ptr(), args[1].data_ptr(),
                      args[2].data_ptr(), args[3].data_ptr(), args[4].data_ptr(),
                      args[5].data_ptr(), 40, args[0].data_ptr(), None, 0, 1, 4, 2, 64, 16,
                      args[3].shape[1], args[1].shape[0], 40, 0.125, 0, 0, 1, None)


def test_captured_decode_survives_workspace_growth(iva, dev):
    """A decode step captured in a HIP graph with the op-owned workspace keeps working
    after a split prefill on the same stream grows that workspace: the smaller one stays
    allocated, so every replay equals the eager decode and memory handed out after the
    growth is never written by the replays."""
    d = iva.workloads.decode_batch([700, 90, 1300], 8, 2, 64, torch.float16, seed=5,
                                   scale=0.125, device=dev)
    lay = d["layout"]
    dargs = (d["q"], d["k_pool"], d["v_pool"], lay.block_tables.to(dev), lay.context_lens.to(dev))
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        eager = iva.paged_decode_attention(*dargs)
        out = torch.empty_like(eager)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            iva.paged_decode_attention(*dargs, out=out)
        c = make(iva, [4000, 2000], [300, 64], 8, 2, 128, torch.float16, seed=7)
        for _ in range(2):  # grows the stream's workspace, then reuses the new one
            iva.paged_prefill_attention(*dev_args(c, dev), split=True)
        junk = torch.full((1 << 24,), 7, dtype=torch.int32, device=dev)  # reuse of freed memory
        for _ in range(3):
            out.zero_()
            g.replay()
            stream.synchronize()
            assert torch.equal(out, eager)
        assert bool((junk == 7).all())
        del junk
    torch.cuda.current_stream(dev).wait_stream(stream)
