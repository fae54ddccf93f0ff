"""Benchmark of the paged KV hot path on one MI355X.

A step is one decode step of the hot path over one batch: append one new K/V row
per sequence into its page, then paged GQA decode attention over the whole
context.  By default the step is the fused op ivakv_decode_append_attn (the paged
walk over the earlier positions + a merge that scores the new token and stores
its rows); --unfused runs ivakv_append then ivakv_decode_attn.
Workload C2: 32 sequences, 32 query / 8 KV heads, head_dim 128, fp16, block 16,
context lengths ~ U[512, 4096] (seed 0), values N(0, 1)/sqrt(128).

Inputs are resident in HBM before timing.  To keep the 256 MiB MALL from
serving repeated reads, steps rotate over --pools independent page pools
(>= 1 GiB in total by default).  Each pool's step is captured once as a HIP
graph (launch overhead of the kernels is then the graph's, as in a production
decode loop) and the graphs are replayed --steps times between two
synchronisations.

Output: one JSON line.  `value` is algorithmic GB/s of the whole step (append
bytes + attention bytes) / step time.  `roofline` is for the dominant kernel
(the paged walk, decode_stream_kernel): its algorithmic bytes / its average
duration measured here with HIP events over a graph of back-to-back launches on
the launch stream.  `cpu_baseline` times the CPU restatement of the reference's
torch path (contiguous cache + torch.cat append + AttentionTorch math, fp32) on
this host's cores.  `target_4k` repeats the walk, attention and step measurements
at the north-star target's own shape (the same batch with every sequence at
context 4096); --no-target-4k skips it, and runs with --eager or
--copy-calibration (the counter runs) never make it.

Profiling helpers (no timing line):
  --copy-calibration   also launches a plain 256 MiB device copy 10 times after
                       the timed region: the known-size kernel that scales the
                       rocprofv3 FETCH_SIZE / WRITE_SIZE counters.
  --summarize-pmc F W  reads the counter CSVs of a FETCH_SIZE run (directory F)
                       and a WRITE_SIZE run (directory W) and writes
                       profiles/decode_attn_c2_traffic.json (with --context N:
                       profiles/decode_attn_ctxN_traffic.json).
  --rdreq-dir R        with --summarize-pmc: a third run's TCC_EA0_RDREQ_{32B,64B,
                       128B}_sum counts, which give the read bytes directly (no copy
                       scale) as a cross-check of the scaled FETCH_SIZE.
"""
from __future__ import annotations

import argparse
import csv
import itertools
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Optional

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode-attn + KV append GB/s and % HBM peak; decode tokens/s at 1 GPU"
def traffic_path(context: str):
    """Committed HBM-traffic summary of the walk for a --context choice (or "c4")."""
    name = context if context in ("c2", "c4") else f"ctx{int(context)}"
    return ROOT / "profiles" / f"decode_attn_{name}_traffic.json"
WALK_KERNEL = "decode_stream_kernel"
COPY_BYTES = 256 << 20


def read_traffic(context: str):
    """HBM bytes per walk launch from the committed counter summary, or None."""
    path = traffic_path(context)
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--pools", type=int, default=4, help="independent KV pools rotated per step")
    p.add_argument("--partition-pages", type=int, default=0,
                   help="0 = default (stream) walk; > 0 = partitioned walk of that size")
    p.add_argument("--kernel-launches", type=int, default=200,
                   help="launches of the paged walk timed for the roofline figure")
    p.add_argument("--cpu-reps", type=int, default=40,
                   help="timed CPU-baseline reps, about 10 s of CPU work at C2 (0 = skip)")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of graphs")
    p.add_argument("--unfused", action="store_true",
                   help="step = ivakv_append + ivakv_decode_attn instead of the fused op")
    p.add_argument("--copy-calibration", action="store_true",
                   help="launch a plain 256 MiB copy 10x after timing (counter calibration)")
    p.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="write the HBM traffic summary from two rocprofv3 --pmc runs")
    p.add_argument("--rdreq-dir", default=None,
                   help="with --summarize-pmc: a run of TCC_EA0_RDREQ_sum and its 32B / 64B / "
                        "128B parts, for read bytes counted by request size")
    p.add_argument("--c5-steps", type=int, default=40, help="timed churn steps of --workload c5")
    p.add_argument("--context", default="c2",
                   help="c2 (default): context lengths U[512, 4096] seed 0 (the contract line); "
                        "an integer N: every sequence of the batch at context N (e.g. 4096, "
                        "the north-star target's 4k context)")
    p.add_argument("--no-target-4k", dest="target_4k", action="store_false",
                   help="skip the second measurement at the target shape (B 32, every "
                        "sequence at context 4096) that the default line carries")
    p.add_argument("--workload", choices=("c2", "c3", "c4", "c5", "prefill", "c2fp8", "ops",
                                          "ceiling"),
                   default="c2",
                   help="c2 (default): the contract line; c3 dense-decoder tokens/s, c4 "
                        "long-context window+sinks decode, c5 ragged churn, prefill: 512-token "
                        "chunks over paged context, c2fp8: C2 over FP8 pages, ops: the append / "
                        "gather / kv_ops / page-move kernels, ceiling: measured streaming "
                        "and random-tile read bandwidth (informational lines)")
    return p.parse_args()


def append_bytes(n_tok, hkv, d, esize):
    """Bytes an append of n_tok rows moves: the K and V rows read (2 n Hkv D esize) and
    written into their slots (as many), plus the int32 slot map.  The one formula of every
    append figure here (the C2 step, the ops and C5 lines); like the gather's, it counts
    reads and writes, twice the rows' size alone."""
    return 4 * n_tok * hkv * d * esize + 4 * n_tok


def algorithmic_bytes(lengths, hq, hkv, d, esize, bs=16):
    """Per-step algorithmic bytes: append of one row per sequence, decode attention."""
    b = len(lengths)
    append = append_bytes(b, hkv, d, esize)
    attn = (sum(2 * n * hkv * d * esize for n in lengths)   # K + V of attended rows
            + 2 * b * hq * d * esize                          # q in, out
            + sum(4 * math.ceil(n / bs) for n in lengths)     # block-table entries
            + 4 * b)                                          # context lengths
    return append, attn


def cpu_baseline(lengths, hq, hkv, d, reps, seed=0):
    """Times the CPU restatement of the reference torch path on a padded fp32 batch."""
    import torch
    from oracle import reference_path as rp

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    b, lmax = len(lengths), max(lengths)
    lens = torch.tensor(lengths)
    sc = 1 / math.sqrt(d)
    ck = torch.randn(b, hkv, lmax - 1, d, generator=g) * sc
    cv = torch.randn(b, hkv, lmax - 1, d, generator=g) * sc
    valid = torch.arange(lmax - 1)[None] < (lens[:, None] - 1)
    q = torch.randn(b, hq, 1, d, generator=g) * sc
    kn = torch.randn(b, hkv, 1, d, generator=g) * sc
    vn = torch.randn(b, hkv, 1, d, generator=g) * sc
    for _ in range(3):
        rp.reference_decode_step(ck, cv, valid, lens, q, kn, vn, sc)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        rp.reference_decode_step(ck, cv, valid, lens, q, kn, vn, sc)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), threads


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _counter_rows(directory: str):
    """(kernel name, counter name, value) of every dispatch in a rocprofv3 --pmc CSV."""
    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {directory}")
    for f in files:
        with f.open() as fh:
            for row in csv.DictReader(fh):
                yield row.get("Kernel_Name", ""), row.get("Counter_Name", ""), float(row["Counter_Value"])


def _mean_kib(directory: str, counter: str, match) -> float:
    vals = [v for k, c, v in _counter_rows(directory) if c == counter and match(k)]
    if not vals:
        raise SystemExit(f"no {counter} rows for the requested kernel in {directory}")
    return sum(vals) / len(vals)


def summarize_pmc(fetch_dir: str, write_dir: str, context: str = "c2",
                  rdreq_dir: Optional[str] = None) -> None:
    """Scales the walk's FETCH_SIZE / WRITE_SIZE (KiB per dispatch) by what the same
    counters read for the plain copy of COPY_BYTES, and writes the traffic summary.
    With rdreq_dir, the read bytes are also counted from the L2's read requests to
    memory by size (32 n32 + 64 n64 + 128 n128 per dispatch), for the walk and for the
    copy: a second counter path that needs no scale."""
    ops = "TileOps<2, 128>" if context == "c4" else "TileOps<1, 128>"   # C4 is bf16
    is_walk = lambda k: WALK_KERNEL in k and ops in k
    is_copy = lambda k: "copy" in k.lower() and "ivakv" not in k

    def copy_kib(directory, counter):
        """The calibration leg's 10 identical copies: the most common (to 2 significant
        digits) large value among copy-kernel dispatches."""
        rows = [v for k, c, v in _counter_rows(directory)
                if c == counter and is_copy(k) and v > 0.25 * COPY_BYTES / 1024]
        if not rows:
            raise SystemExit(f"no calibration copy rows for {counter} in {directory}")
        key = lambda v: float(f"{v:.2g}")
        groups = {}
        for v in rows:
            groups.setdefault(key(v), []).append(v)
        best = max(groups.values(), key=len)
        return sum(best) / len(best)
    fetch_walk = _mean_kib(fetch_dir, "FETCH_SIZE", is_walk)
    write_walk = _mean_kib(write_dir, "WRITE_SIZE", is_walk)
    fetch_copy = copy_kib(fetch_dir, "FETCH_SIZE")
    write_copy = copy_kib(write_dir, "WRITE_SIZE")
    f_scale = COPY_BYTES / (fetch_copy * 1024)
    w_scale = COPY_BYTES / (write_copy * 1024)
    read_b = fetch_walk * 1024 * f_scale
    write_b = write_walk * 1024 * w_scale
    summary = {
        "kernel": ("decode_stream_kernel<bf16,128> (C4)" if context == "c4" else
                   "decode_stream_kernel<f16,128> (%s)" % (
                       "C2" if context == "c2" else f"B 32 at context {int(context)}")),
        "fetch_kib_per_dispatch": round(fetch_walk, 1),
        "write_kib_per_dispatch": round(write_walk, 1),
        "copy_calibration_bytes": COPY_BYTES,
        "copy_fetch_kib": round(fetch_copy, 1),
        "copy_write_kib": round(write_copy, 1),
        "fetch_scale": round(f_scale, 4),
        "write_scale": round(w_scale, 4),
        "hbm_read_bytes_per_launch": int(read_b),
        "hbm_write_bytes_per_launch": int(write_b),
        "hbm_bytes_per_launch": int(read_b + write_b),
    }
    if rdreq_dir:
        def rdreq(match):
            parts = {}
            for size in ("", "_32B", "_64B", "_128B"):
                name = f"TCC_EA0_RDREQ{size}_sum"
                vals = [v for k, c, v in _counter_rows(rdreq_dir) if c == name and match(k)]
                if not vals:
                    raise SystemExit(f"no {name} rows in {rdreq_dir}")
                parts[size or "all"] = vals
            return parts
        walk = {k: sum(v) / len(v) for k, v in rdreq(is_walk).items()}
        # the copy: dispatches whose 128-byte requests cover at least a quarter of it
        copy_all = rdreq(is_copy)
        big = [i for i, v in enumerate(copy_all["_128B"]) if v * 128 > 0.25 * COPY_BYTES]
        if not big:
            raise SystemExit(f"no calibration copy rows in {rdreq_dir}")
        copy = {k: sum(v[i] for i in big) / len(big) for k, v in copy_all.items()}
        by_size = lambda d: 32 * d["_32B"] + 64 * d["_64B"] + 128 * d["_128B"]
        summary.update({
            "rdreq_walk": {k: round(v, 1) for k, v in walk.items()},
            "rdreq_copy": {k: round(v, 1) for k, v in copy.items()},
            "rdreq_read_bytes_per_launch": int(by_size(walk)),
            "rdreq_copy_read_bytes": int(by_size(copy)),
            "rdreq_over_scaled_fetch": round(by_size(walk) / read_b, 4),
        })
    out = traffic_path(context)
    out.parent.mkdir(exist_ok=True)
    out.write_text(json.dumps(summary, indent=1) + "\n")
    print(json.dumps(summary))


def _ceiling_lib():
    """The read-ceiling kernels (iva1.0_amd/bench_kernels/ivakv_ceiling.hip), built by
    build() into libivakv_ceiling.so."""
    import ctypes
    path = ROOT / "iva1.0_amd" / "libivakv_ceiling.so"
    if not path.exists():
        raise SystemExit(f"{path} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(path))
    c_int, c_int64, c_void_p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
    lib.ceiling_stream.argtypes = [c_void_p, c_int64, c_void_p, c_int, c_int, c_int, c_void_p]
    lib.ceiling_tiles.argtypes = [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p,
                                  c_int, c_void_p]
    lib.ceiling_mfma.argtypes = [c_int, c_void_p, c_void_p, c_int, c_void_p]
    return lib


STREAM_WG_PER_CU = (1, 2, 4, 8)
STREAM_PER_LANE = (4, 8)
TILE_WG_PER_CU = (1, 2, 4)
TILE_RING = (2, 4)


def measure_ceiling(torch, dev, sets=4, set_bytes=288 << 20, tile_bytes=4096,
                    tiles_per_launch=70144, reps=40):
    """Read-bandwidth reference points of this GPU, on 4 rotated buffers of 288 MiB (as
    the C2 bench rotates its pools), each the best over a sweep of launch shapes:
    - stream: each wave reads its own contiguous share, 4 or 8 16-byte loads per lane
      per slot with two slots in flight (8 or 16 KiB per wave), at 1 / 2 / 4 / 8 4-wave
      workgroups per CU, with and without the non-temporal hint;
    - tiles: tiles_per_launch random 4 KiB tiles of each buffer (the C2 walk's 70,144 K
      and V tiles), 2 or 4 tiles in flight per wave (4 = the walk's 16 KiB), 1 / 2 / 4
      workgroups per CU, with and without the hint.
    GB/s = bytes read / average launch time over back-to-back launches (HIP events).
    These are measured reference points for the access patterns, not hardware limits."""
    lib = _ceiling_lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    gen = torch.Generator().manual_seed(3)
    bufs = [torch.empty(set_bytes, dtype=torch.uint8, device=dev).fill_(i + 1) for i in range(sets)]
    n_tiles = set_bytes // tile_bytes
    idxs = [torch.randperm(n_tiles, generator=gen)[:tiles_per_launch].to(torch.int32).to(dev)
            for _ in range(sets)]
    sink = torch.empty(cus * 8 * 4 * 16, dtype=torch.uint8, device=dev)   # one word per wave

    def timed(launch):
        for i in range(sets):
            launch(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for r in range(reps):
            launch(r % sets)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) * 1e-3 / reps

    def check(rc):
        if rc != 0:
            raise SystemExit(f"ceiling kernel launch failed ({rc})")

    stream_gbs = {}
    for per_cu, per_lane, nt in itertools.product(STREAM_WG_PER_CU, STREAM_PER_LANE, (0, 1)):
        t = timed(lambda i: check(lib.ceiling_stream(bufs[i].data_ptr(), set_bytes,
                                                     sink.data_ptr(), cus * per_cu, per_lane,
                                                     nt, st)))
        stream_gbs[f"wg{per_cu}_u{per_lane}_nt{nt}"] = set_bytes / t / 1e9
    tile_gbs = {}
    for per_cu, ring, nt in itertools.product(TILE_WG_PER_CU, TILE_RING, (0, 1)):
        t = timed(lambda i: check(lib.ceiling_tiles(bufs[i].data_ptr(), idxs[i].data_ptr(),
                                                    tiles_per_launch, tile_bytes, ring, nt,
                                                    sink.data_ptr(), cus * per_cu, st)))
        tile_gbs[f"wg{per_cu}_ring{ring}_nt{nt}"] = tiles_per_launch * tile_bytes / t / 1e9
    del bufs, idxs
    mfma_tf = measure_mfma(torch, dev)
    s_best = max(stream_gbs, key=stream_gbs.get)
    t_best = max(tile_gbs, key=tile_gbs.get)
    return {"stream_read_gbs": round(stream_gbs[s_best], 1), "stream_read_best": s_best,
            "stream_read_gbs_by_shape": {k: round(v, 1) for k, v in stream_gbs.items()},
            "tile_read_gbs": round(tile_gbs[t_best], 1), "tile_read_best": t_best,
            "tile_read_gbs_by_shape": {k: round(v, 1) for k, v in tile_gbs.items()},
            "read_reference_gbs": round(max(stream_gbs[s_best], tile_gbs[t_best]), 1),
            "mfma_f16_tflops": round(max(mfma_tf.values()), 1),
            "mfma_f16_tflops_by_waves_per_simd": {k: round(v, 1) for k, v in mfma_tf.items()},
            "sample": f"{sets} rotated buffers of {set_bytes >> 20} MiB; stream: wg{{1,2,4,8}} "
                      f"4-wave workgroups per CU x u{{4,8}} 16-byte loads per lane per slot "
                      f"(2 slots in flight) x nt{{0,1}} non-temporal hint; tiles: "
                      f"{tiles_per_launch} random {tile_bytes}-byte tiles per launch, "
                      f"wg{{1,2,4}} x ring{{2,4}} tiles in flight per wave x nt{{0,1}} "
                      f"({cus} CUs); best shape reported"}


def measure_mfma(torch, dev, iters=20000, reps=5):
    """Dense fp16 MFMA throughput of this GPU (TFLOP/s by waves per SIMD): 1 / 2 / 4
    4-wave workgroups per CU, each wave 8 independent chains of `iters` 16x16x32 MFMAs
    (the prefill's instruction) on random N(0, 0.5) fp16 operands read once, with no
    memory traffic in the loop; average over back-to-back launches (HIP events)."""
    lib = _ceiling_lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev)
    sink = torch.empty(cus * 16 * 16, dtype=torch.uint8, device=dev)   # one word per wave
    gen = torch.Generator(device=dev).manual_seed(11)
    ops = (torch.randn(1024 * 4 * 64 * 8, generator=gen, device=dev) * 0.5).half()
    out = {}
    for per_cu in (1, 2, 4):
        launch = lambda: lib.ceiling_mfma(iters, ops.data_ptr(), sink.data_ptr(), cus * per_cu,
                                          stream.cuda_stream)
        if launch() != 0:
            raise SystemExit("ceiling_mfma launch failed")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        t = e0.elapsed_time(e1) * 1e-3 / reps
        out[per_cu] = cus * per_cu * 4 * iters * 8 * 16384 / t / 1e12
    return out


def bench_ceiling(args, iva, torch, dev):
    """Measured read and MFMA ceilings of the GPU (see measure_ceiling, measure_mfma)."""
    c = measure_ceiling(torch, dev)
    return {"metric": "HBM read ceiling GB/s (streaming and random 4 KiB tiles); dense fp16 MFMA TFLOP/s",
            "workload": "ceiling", "value": c["read_reference_gbs"], "unit": "GB/s",
            "peak": HBM_PEAK_GBS, **c}


def _timer(torch, dev):
    def measure(fn, reps=1):
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / reps * 1e-3
    return measure


def bench_c3(args, iva, torch, dev):
    """C3: dense decoder (d 1024, 16 layers, 16 heads, head_dim 64, vocab 32000, RMSNorm +
    SwiGLU, random init, bf16), 16 prompts of 512 uniform-random ids + 256 greedy steps
    on the paged cache.  Decode tokens/s come from the difference of two generate()
    calls (256 and 128 new tokens), so prefill and graph capture cancel out."""
    M = iva.model
    measure = _timer(torch, dev)
    cfg = M.TransformerConfig(d_model=1024, n_layers=16, n_heads=16, vocab_size=32000,
                              seq_len=4096, attn_impl="hip_paged", dropout=0.0)
    torch.manual_seed(0)
    model = M.Transformer(cfg).to(dev, torch.bfloat16).eval()
    prompts = torch.randint(0, 32000, (16, 512), generator=torch.Generator().manual_seed(0)).to(dev)
    gen = lambda n, graph: model.generate(prompts, max_length=n, do_sample=False,
                                          eos_token_id=None, use_graph=graph)
    with torch.no_grad():
        gen(4, True)
        gen(4, False)

        def prefill():
            cache = model.new_kv_cache(16, 512 + 256)
            model(prompts, kv_cache=cache)
            cache.free()
        t_prefill = measure(prefill, 3)
        t256 = measure(lambda: gen(256, True))
        t128 = measure(lambda: gen(128, True))
        e64 = measure(lambda: gen(64, False))
        e32 = measure(lambda: gen(32, False))
        tokens_paged = gen(256, True)
        ref = M.Transformer(M.TransformerConfig(**{**cfg.__dict__, "attn_impl": "torch"})).to(
            dev, torch.bfloat16).eval()
        ref.load_state_dict(model.state_dict())
        tokens_torch = ref.generate(prompts, max_length=256, do_sample=False, eos_token_id=None)
        same = (tokens_paged == tokens_torch)[:, 512:]
        first_diff = [int((~row).nonzero()[0]) if (~row).any() else 256 for row in same.cpu()]
        # The torch backend's top-2 logit margin where each sequence first diverges,
        # teacher-forced along its own stream (one causal forward): a divergence is a
        # near-tie when that margin is within twice the logits' bf16 agreement bound.
        logits = ref(tokens_torch[:, :-1])["logits"]
        margins = []
        for b, s in enumerate(first_diff):
            if s < 256:
                top = logits[b, 511 + s].float().topk(2).values
                margins.append(round(float(top[0] - top[1]), 4))
            else:
                margins.append(None)
        del logits
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    step_s = (t256 - t128) / 128
    return {
        "metric": "C3 dense-decoder greedy decode tokens/s (paged KV, bf16)", "workload": "c3",
        "value": round(16 / step_s, 1), "unit": "tokens/s", "n_gpus": 1, "dtype": "bf16",
        "data": "synthetic (random init, uniform-random prompt ids)",
        "config": {"d_model": 1024, "n_layers": 16, "n_heads": 16, "head_dim": 64,
                   "vocab": 32000, "batch": 16, "prompt": 512, "new_tokens": 256,
                   "launch": "decode step captured as one HIP graph"},
        "ms_per_decode_step": round(step_s * 1e3, 4),
        "eager_tokens_per_s": round(16 * 32 / (e64 - e32), 1),
        "prefill_ms": round(t_prefill * 1e3, 3),
        "end_to_end_tokens_per_s": round(16 * 256 / (t256 - t_prefill), 1),
        "weight_bytes": weight_bytes,
        "weights_gbps_per_step": round(weight_bytes / step_s / 1e9, 1),
        "greedy_tokens_identical_to_torch_backend": int(same.all(dim=1).sum()),
        "first_divergence_per_seq": first_diff,
        "torch_top2_margin_at_first_divergence": margins,
        # twice the teacher-forced logit bound of tests/test_c3_model_gpu.py (0.09375)
        "near_tie_margin": 0.1875,
    }


def bench_c2fp8(args, iva, torch, dev):
    """C2's batch (B 32, GQA 32/8, D 128, context U[512, 4096] seed 0) over FP8 (e4m3fn)
    pages with per-(slot, kv head) scaling factors; fp16 queries.  GB/s on the bytes the
    FP8 walk must move (codes, factors, q, out, tables) and decode tokens/s, beside the
    fp16-page attention of the same batch."""
    wl = iva.workloads
    measure = _timer(torch, dev)
    hq, hkv, d = 32, 8, 128
    lengths = wl.c2_lengths(seed=0)
    batch = len(lengths)
    sc = 1 / math.sqrt(d)
    sets8, sets16 = [], []
    for i in range(args.pools):
        dd = wl.decode_batch(lengths, hq, hkv, d, torch.float16, seed=100 + i, device=dev, scale=sc)
        lay = dd["layout"]
        bt, ctx = lay.block_tables.to(dev), lay.context_lens.to(dev)
        ks, vs = iva.pool_shapes(lay.num_pages, hkv, d, 16, torch.float8_e4m3fn)
        k8 = torch.zeros(ks, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        v8 = torch.zeros(vs, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        kss = torch.ones(iva.scale_shape(lay.num_pages, hkv), device=dev)
        vss = torch.ones_like(kss)
        kc, vc = iva.kv_gather(dd["k_pool"], dd["v_pool"], bt, ctx)  # the fp16 rows, re-paged
        slots = torch.cat([lay.slots(b, torch.arange(n)) for b, n in enumerate(lengths)]).to(dev)
        rows_k = torch.cat([kc[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)])
        rows_v = torch.cat([vc[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)])
        iva.kv_append(rows_k, rows_v, k8, v8, slots, k_scale=kss, v_scale=vss)
        del kc, vc, rows_k, rows_v
        q, out = dd["q"], torch.empty_like(dd["q"])
        gen = torch.Generator(device=dev).manual_seed(500 + i)
        kn = (torch.randn(batch, hkv, d, generator=gen, device=dev) * sc).half()
        vn = (torch.randn(batch, hkv, d, generator=gen, device=dev) * sc).half()
        last = torch.stack([lay.slots(b, torch.tensor([n - 1])) for b, n in enumerate(lengths)])
        sets8.append((q, k8, v8, bt, ctx, out, kss, vss, kn, vn, last.reshape(-1).to(dev)))
        sets16.append((q, dd["k_pool"], dd["v_pool"], bt, ctx, out))
    ws = torch.empty(iva.decode_workspace_bytes(batch, hq, hkv, d, 16, sets8[0][3].shape[1]),
                     dtype=torch.uint8, device=dev)
    run8 = lambda s: iva.paged_decode_attention(s[0], s[1], s[2], s[3], s[4], out=s[5],
                                                workspace=ws, k_scale=s[6], v_scale=s[7])
    run16 = lambda s: iva.paged_decode_attention(s[0], s[1], s[2], s[3], s[4], out=s[5],
                                                 workspace=ws)
    # decode steps on FP8 pages: the new row of every sequence (position L-1) appended
    # and attended, in one op (ivakv_decode_append_attn_fp8) or as append + attention
    step8 = lambda s: iva.paged_decode_append_attention(
        s[0], s[8], s[9], s[1], s[2], s[3], s[4], out=s[5], workspace=ws, k_scale=s[6],
        v_scale=s[7])

    def step8_unfused(s):
        iva.kv_append(s[8], s[9], s[1], s[2], s[10], k_scale=s[6], v_scale=s[7])
        run8(s)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    reps = 20
    with torch.cuda.stream(stream):
        for s in sets8:
            run8(s)
            step8(s)
            step8_unfused(s)
        for s in sets16:
            run16(s)
        torch.cuda.synchronize(dev)
        graphs = []
        for fn, sets in ((run8, sets8), (run16, sets16), (step8, sets8), (step8_unfused, sets8)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for r in range(reps):
                    fn(sets[r % len(sets)])
            graphs.append(g)
        times = []
        for g in graphs:
            g.replay()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(10):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize(dev)
            times.append(e0.elapsed_time(e1) * 1e-3 / (10 * reps))
    t8, t16, ts8, ts8u = times
    tokens = sum(lengths)
    byts = 2 * tokens * hkv * d + 2 * tokens * hkv * 4 + 2 * batch * hq * d * 2 + \
        sum(-(-n // 16) for n in lengths) * 4 + 4 * batch
    return {"metric": "C2 decode attention over FP8 pages GB/s (codes + factors) and tokens/s",
            "workload": "c2fp8", "value": round(byts / t8 / 1e9, 1), "unit": "GB/s",
            "dtype": "fp8 e4m3fn pages, f16 q/out",
            "config": {"batch": batch, "heads": "32/8", "head_dim": d, "context": "U[512,4096] seed 0",
                       "launch": "hip graph", "walk": "stream"},
            "attention_us": round(t8 * 1e6, 2), "fp16_pages_attention_us": round(t16 * 1e6, 2),
            "speedup_vs_fp16_pages": round(t16 / t8, 3), "bytes": byts,
            "tokens_per_s": round(batch / t8, 1),
            "step_us": round(ts8 * 1e6, 2), "step_unfused_us": round(ts8u * 1e6, 2),
            "step_ops": "ivakv_decode_append_attn_fp8 (fused); unfused: ivakv_append_fp8 + "
                        "ivakv_decode_attn_fp8"}


C4_RESIDENT_POOLS = 16


def bench_c4(args, iva, torch, dev):
    """C4: long-context decode, bf16, B 4 at 32k/64k/96k/128k, GQA 32/8, D 128, window
    4096 + 4 sinks (union); GB/s on attended bytes.  The pools are what a sliding-window
    PagedKVCache keeps resident (the sink pages and the window's; the rest released after
    each forward): 67.6 MB each, so 16 of them are rotated (1.08 GB) for the MALL not to
    serve repeats.  Attention (walk + merge) and the walk alone, each as a HIP graph of
    back-to-back launches over the rotated pools, plus the same eagerly."""
    wl = iva.workloads
    measure = _timer(torch, dev)
    sets = []
    n_pools = max(args.pools, C4_RESIDENT_POOLS)
    for i in range(n_pools):
        d = wl.c4_long_context(seed=10 + i, device=dev, resident_window=True)
        lay = d["layout"]
        sets.append((d["q"], d["k_pool"], d["v_pool"], lay.block_tables.to(dev),
                     lay.context_lens.to(dev), torch.empty_like(d["q"])))
    resident = sets[0][1].numel() * sets[0][1].element_size() * 2
    full_pages = sum(math.ceil(n / 16) for n in wl.C4_LENGTHS)
    full_bytes = full_pages * 8 * 128 * 16 * 2 * 2
    w, ns = wl.C4_WINDOW, wl.C4_SINKS
    batch, max_blocks = sets[0][0].shape[0], sets[0][3].shape[1]
    ws = torch.empty(iva.decode_workspace_bytes(batch, 32, 8, 128, 16, max_blocks, w, ns),
                     dtype=torch.uint8, device=dev)
    run = lambda s, fn: fn(s[0], s[1], s[2], s[3], s[4], window=w, n_sink=ns, out=s[5],
                           workspace=ws)
    attn = lambda s: run(s, iva.paged_decode_attention)
    walk = lambda s: run(s, iva.paged_decode_attention_partial)
    reps = 48
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for s in sets:
            attn(s)
            walk(s)
        torch.cuda.synchronize(dev)

        def graph_us(fn):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for r in range(reps):
                    fn(sets[r % len(sets)])
            g.replay()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(4):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize(dev)
            return e0.elapsed_time(e1) * 1e3 / (4 * reps)
        t_attn, t_walk = graph_us(attn), graph_us(walk)
        e_attn = measure(lambda: [attn(sets[i % len(sets)]) for i in range(reps)]) / reps * 1e6
        e_walk = measure(lambda: [walk(sets[i % len(sets)]) for i in range(reps)]) / reps * 1e6
    if args.copy_calibration:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(7)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
    attended = [min(n, w) + min(ns, max(n - w, 0)) for n in wl.C4_LENGTHS]
    byts = sum(2 * a * 8 * 128 * 2 for a in attended) + 2 * 4 * 32 * 128 * 2
    return {"metric": "C4 long-context windowed decode attention GB/s (attended bytes)",
            "workload": "c4", "value": round(byts / (t_attn * 1e-6) / 1e9, 1), "unit": "GB/s",
            "dtype": "bf16", "config": {"lengths": wl.C4_LENGTHS, "window": w, "sinks": ns,
                                        "heads": "32/8", "head_dim": 128,
                                        "launch": "hip graph of back-to-back launches",
                                        "pools_rotated": n_pools,
                                        "pool": "resident window: sink + window pages only"},
            "resident_bytes": resident, "full_context_bytes": full_bytes,
            "attention_us": round(t_attn, 2), "walk_us": round(t_walk, 2),
            "walk_gbps": round(byts / (t_walk * 1e-6) / 1e9, 1),
            "walk_frac": round(byts / (t_walk * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "eager_attention_us": round(e_attn, 2), "eager_walk_us": round(e_walk, 2),
            "attended_bytes": byts, "traffic": read_traffic("c4")}


C5_PER_GRAPH = 4   # launches of one C5 op per captured graph


def bench_c5(args, iva, torch, dev):
    """C5: ragged continuous-batching churn, fp16, GQA 32/8, D 128: 256 live sequences of
    total length LogNormal(ln 1024, sigma 1) capped at 16k, the last U{1..256} tokens
    decoded one per step after 512-token prefill chunks, completed sequences replaced
    (LIFO page reuse), every sequence starting at a random point of its lifetime
    (workloads.ChurnBatch).  A step appends every prefill chunk (ivakv_append), runs the
    chunks' causal attention over their pages (ivakv_prefill_attn) and the decode step of
    every decoding sequence (append + attention, ivakv_decode_append_attn).  Each of the
    three is timed on the GPU as launches back to back inside one captured HIP graph
    (C5_PER_GRAPH per graph, the graph replayed `reps` times, so a short op's time is not
    the graph launch's), with the step's inputs already on the device; the step time is
    their sum."""
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    wl = iva.workloads
    hq, hkv, d, sc = 32, 8, 128, 128 ** -0.5
    pool = pc.PagedKVPool(64000, hkv, d, 16, 1, torch.float16, dev, max_seqs=512,
                          max_blocks_per_seq=1024)
    churn = wl.ChurnBatch(pool, n_seqs=256, seed=0, scale=sc)
    gen = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *shape: (torch.randn(*shape, generator=gen, device=dev) * sc).half()
    ws = torch.empty(iva.decode_workspace_bytes(256, hq, hkv, d, 16, pool.max_blocks),
                     dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    reps = 5
    rows = {k: [] for k in ("append_us", "prefill_us", "decode_us", "step_us", "chunk_tok",
                            "decode_seqs", "decode_bytes", "append_bytes", "prefill_flop",
                            "completed", "mean_context")}
    for step in range(5 + args.c5_steps):
        plan = churn.plan_step()
        pre_ids = [sid for sid, _ in plan["prefill"]]
        n_chunk = len(plan["prefill_slots"])
        dec_ids = plan["decode"]
        kc, vc, qc = rnd(n_chunk, hkv, d), rnd(n_chunk, hkv, d), rnd(n_chunk, hq, d)
        slots = torch.from_numpy(plan["prefill_slots"]).to(dev)
        qs = torch.tensor(list(itertools.accumulate([n for _, n in plan["prefill"]],
                                                    initial=0)), dtype=torch.int32, device=dev)
        bt_p, ctx_p = churn.tables(pre_ids) if pre_ids else (None, None)
        bt_d, ctx_d = churn.tables(dec_ids)
        qd, kd, vd = rnd(len(dec_ids), hq, d), rnd(len(dec_ids), hkv, d), rnd(len(dec_ids), hkv, d)
        out_d = torch.empty_like(qd)
        max_chunk = max((n for _, n in plan["prefill"]), default=0)
        out_p = torch.empty_like(qc)
        ops = {"append": lambda: iva.kv_append(kc, vc, pool.k_pools[0], pool.v_pools[0], slots),
               "prefill": lambda: iva.paged_prefill_attention(
                   qc, pool.k_pools[0], pool.v_pools[0], bt_p, ctx_p, qs,
                   max_query_len=max_chunk, out=out_p),
               "decode": lambda: iva.paged_decode_append_attention(
                   qd, kd, vd, pool.k_pools[0], pool.v_pools[0], bt_d, ctx_d, out=out_d,
                   workspace=ws)}
        if not n_chunk:
            del ops["append"], ops["prefill"]
        # Each op is captured C5_PER_GRAPH times into one HIP graph, replayed once (the
        # step), then replayed back to back for its GPU time: the ops are idempotent (the
        # same rows to the same slots; attention rewrites its output), so the repeats
        # leave the step's state as one run does.
        t_op = {}
        stream.wait_stream(torch.cuda.current_stream(dev))   # the step's inputs
        with torch.cuda.stream(stream):
            graphs = {}
            for name, fn in ops.items():
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    for _ in range(C5_PER_GRAPH):
                        fn()
                graphs[name] = g
            for g in graphs.values():
                g.replay()
            for name, g in graphs.items():
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    g.replay()
                e1.record(stream)
                torch.cuda.synchronize(dev)
                t_op[name] = e0.elapsed_time(e1) * 1e3 / (reps * C5_PER_GRAPH)
        del graphs
        dec_lens = churn.lengths(dec_ids)
        pre_lens = churn.lengths(pre_ids)
        done = churn.finish_step()
        if step < 5:
            continue
        rows["append_us"].append(t_op.get("append", 0.0))
        rows["prefill_us"].append(t_op.get("prefill", 0.0))
        rows["decode_us"].append(t_op["decode"])
        rows["step_us"].append(sum(t_op.values()))
        rows["chunk_tok"].append(n_chunk)
        rows["decode_seqs"].append(len(dec_ids))
        rows["decode_bytes"].append(sum(2 * n * hkv * d * 2 for n in dec_lens)
                                    + 2 * len(dec_ids) * hq * d * 2)
        rows["append_bytes"].append(append_bytes(n_chunk, hkv, d, 2))
        rows["prefill_flop"].append(sum(4 * d * hq * sum(range(L - n + 1, L + 1))
                                        for (_, n), L in zip(plan["prefill"], pre_lens)))
        rows["completed"].append(done)
        rows["mean_context"].append(statistics.mean(churn.lengths()))
    med = lambda k: statistics.median(rows[k])
    dec_gbs = statistics.median([b / (x * 1e-6) / 1e9 for b, x in zip(rows["decode_bytes"], rows["decode_us"])])
    app_gbs = statistics.median([b / (x * 1e-6) / 1e9 for b, x in zip(rows["append_bytes"], rows["append_us"]) if x > 0])
    pre_tf = statistics.median([f / (x * 1e-6) / 1e12 for f, x in zip(rows["prefill_flop"], rows["prefill_us"]) if x > 0])
    return {"metric": "C5 ragged churn: decode step (append + attention) GB/s per step",
            "workload": "c5", "value": round(dec_gbs, 1), "unit": "GB/s", "dtype": "f16",
            "config": {"live_seqs": 256, "lengths": "total LogNormal(ln 1024, 1.0) capped 16384",
                       "generated": "U{1..256} tokens per sequence, one per step",
                       "prefill_chunk": 512, "steps": args.c5_steps, "heads": "32/8",
                       "head_dim": 128,
                       "launch": f"each op {C5_PER_GRAPH} launches per HIP graph, replayed back to back, inputs on the device"},
            "step_us_median": round(med("step_us"), 1),
            "steps_per_s": round(1e6 / med("step_us"), 1),
            "decode_us_median": round(med("decode_us"), 1),
            "decode_seqs_median": med("decode_seqs"),
            "append_us_median": round(med("append_us"), 1),
            "append_gbps": round(app_gbs, 1),
            "prefill_us_median": round(med("prefill_us"), 1),
            "prefill_tflops": round(pre_tf, 1),
            "prefill_chunk_tokens_median": med("chunk_tok"),
            "completions_per_step_mean": round(statistics.mean(rows["completed"]), 2),
            "steps_with_completions": sum(1 for c in rows["completed"] if c),
            "mean_context": round(statistics.mean(rows["mean_context"]), 1),
            "lognormal_mean": round(churn.lognormal_mean(), 1),
            "free_pages_left": pool.num_free_pages}


def bench_prefill(args, iva, torch, dev):
    """Chunked prefill at C5's chunk size: 16 sequences each appending a 512-token chunk
    on top of 1536 cached positions (context 2048), GQA 32/8, D 128, fp16.  TFLOP/s on
    algorithmic causal FLOPs: 4 * D * Hq * (visible keys) summed over query rows.  The
    value is the op's default path (split, by its work bound); the single-launch kernel,
    FP8 pages and two long-context batches (one 512-token chunk at 16k keys; chunks at
    4k / 8k / 16k / 32k) are reported beside it, each split and single-launch."""
    wl = iva.workloads
    measure = _timer(torch, dev)
    hq, hkv, d = 32, 8, 128
    reps = 40

    def batch_sets(lengths, chunks, n_sets, seed):
        out = []
        for i in range(n_sets):
            c = wl.prefill_batch(lengths, chunks, hq, hkv, d, torch.float16, seed=seed + i,
                                 device=dev, scale=d ** -0.5)
            lay = c["layout"]
            out.append((c["q"], c["k_pool"], c["v_pool"], lay.block_tables.to(dev),
                        lay.context_lens.to(dev), c["query_start"].to(dev),
                        torch.empty_like(c["q"])))
        return out

    def time_sets(sets, max_q, split, n=reps, **kw):
        # an untimed pass (clocks, caches), then the better of two timed passes
        run = lambda s: iva.paged_prefill_attention(s[0], s[1], s[2], s[3], s[4], s[5],
                                                    max_query_len=max_q, out=s[6], split=split,
                                                    **kw)
        batch = lambda: [run(sets[i % len(sets)]) for i in range(n)]
        batch()
        return min(measure(batch), measure(batch)) / n

    def tflops(lengths, chunks):
        return sum(4 * d * hq * (L - n + i + 1) for L, n in zip(lengths, chunks) for i in range(n))

    lengths, chunks = [2048] * 16, [512] * 16
    sets = batch_sets(lengths, chunks, args.pools, 20)
    t = time_sets(sets, 512, None)
    t_single = time_sets(sets, 512, False)
    t_split = time_sets(sets, 512, True)
    # the same batch over FP8 pages (the fp16 rows quantized by the FP8 append)
    sets8 = []
    for s in sets:
        lay_pages = s[1].shape[0]
        ks, vs = iva.pool_shapes(lay_pages, hkv, d, 16, torch.float8_e4m3fn)
        k8 = torch.zeros(ks, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        v8 = torch.zeros(vs, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        kss = torch.ones(iva.scale_shape(lay_pages, hkv), device=dev)
        vss = torch.ones_like(kss)
        kc, vc = iva.kv_gather(s[1], s[2], s[3], s[4])
        slots = torch.cat([(s[3][b, torch.arange(n, device=dev) // 16].long() * 16 +
                            torch.arange(n, device=dev) % 16) for b, n in enumerate(lengths)])
        rows_k = torch.cat([kc[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)])
        rows_v = torch.cat([vc[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)])
        iva.kv_append(rows_k, rows_v, k8, v8, slots.int(), k_scale=kss, v_scale=vss)
        del kc, vc, rows_k, rows_v
        sets8.append((s[0], k8, v8, s[3], s[4], s[5], s[6], kss, vss))
    run8 = lambda s: iva.paged_prefill_attention(s[0], s[1], s[2], s[3], s[4], s[5],
                                                 max_query_len=512, out=s[6], k_scale=s[7],
                                                 v_scale=s[8])
    batch8 = lambda: [run8(sets8[i % len(sets8)]) for i in range(reps)]
    batch8()
    t8 = min(measure(batch8), measure(batch8)) / reps
    del sets8
    flops = tflops(lengths, chunks)
    tf = flops / t / 1e12
    long_ctx = {}
    for name, (ll, cc) in {"one_chunk_at_16k": ([16384], [512]),
                           "chunks_at_4k_8k_16k_32k": ([4096, 8192, 16384, 32768], [512] * 4)}.items():
        lsets = batch_sets(ll, cc, 2, 60)
        f = tflops(ll, cc)
        ts, t1 = time_sets(lsets, 512, True, 10), time_sets(lsets, 512, False, 10)
        long_ctx[name] = {"split_us": round(ts * 1e6, 1), "split_tflops": round(f / ts / 1e12, 1),
                          "single_launch_us": round(t1 * 1e6, 1),
                          "single_launch_tflops": round(f / t1 / 1e12, 1)}
        del lsets
    mfma_ceiling = max(measure_mfma(torch, dev).values())
    return {"metric": "paged chunked-prefill attention TFLOP/s", "workload": "prefill",
            "value": round(tf, 1), "unit": "TFLOP/s", "dtype": "f16",
            "config": {"sequences": 16, "chunk": 512, "context": 2048, "heads": "32/8",
                       "head_dim": 128, "launch": "eager", "path": "default (split)"},
            "kernel_us": round(t * 1e6, 2), "algorithmic_flops": flops,
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                         "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4)},
            "measured_mfma_f16_ceiling_tflops": round(mfma_ceiling, 1),
            "frac_of_measured_mfma_ceiling": round(tf / mfma_ceiling, 4),
            "single_launch_kernel_us": round(t_single * 1e6, 2),
            "split_kernel_us": round(t_split * 1e6, 2),
            "fp8_pages_kernel_us": round(t8 * 1e6, 2),
            "fp8_pages_tflops": round(flops / t8 / 1e12, 1),
            "long_context": long_ctx}


def measure_decode(args, iva, torch, dev, lengths):
    """Times the C2-shaped decode step (fused append + attention), the walk and the
    attention over ``lengths`` on rotated pools: HIP graphs of back-to-back launches on
    one stream.  Returns step ms, walk and attention µs per launch, and the pool bytes."""
    wl = iva.workloads
    hq, hkv, d, dtype, esize = 32, 8, 128, torch.float16, 2
    batch = len(lengths)
    sc = 1 / math.sqrt(d)
    sets = []
    for i in range(args.pools):
        dd = wl.decode_batch(lengths, hq, hkv, d, dtype, seed=100 + i, device=dev, scale=sc)
        lay = dd["layout"]
        bt = lay.block_tables.to(dev)
        ctx = lay.context_lens.to(dev)
        pos = torch.tensor([n - 1 for n in lengths])
        slots = torch.stack([lay.slots(b, pos[b]) for b in range(batch)]).to(dev)
        gen = torch.Generator(device=dev).manual_seed(500 + i)
        k_new = (torch.randn(batch, hkv, d, generator=gen, device=dev) * sc).to(dtype)
        v_new = (torch.randn(batch, hkv, d, generator=gen, device=dev) * sc).to(dtype)
        sets.append(dict(q=dd["q"], k_pool=dd["k_pool"], v_pool=dd["v_pool"], bt=bt, ctx=ctx,
                         slots=slots, k_new=k_new, v_new=v_new, out=torch.empty_like(dd["q"])))
    pool_bytes = sum(s["k_pool"].numel() * esize * 2 for s in sets)
    max_blocks = sets[0]["bt"].shape[1]
    ws_bytes = iva.decode_workspace_bytes(batch, hq, hkv, d, 16, max_blocks,
                                          partition_pages=args.partition_pages)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    pp = args.partition_pages or None

    def attention(s):
        iva.paged_decode_attention(s["q"], s["k_pool"], s["v_pool"], s["bt"], s["ctx"],
                                   partition_pages=pp, out=s["out"], workspace=workspace)

    def step(s):
        if args.unfused or args.partition_pages:
            iva.kv_append(s["k_new"], s["v_new"], s["k_pool"], s["v_pool"], s["slots"])
            attention(s)
        else:  # append + attend in one op (ivakv_decode_append_attn)
            iva.paged_decode_append_attention(s["q"], s["k_new"], s["v_new"], s["k_pool"],
                                              s["v_pool"], s["bt"], s["ctx"], out=s["out"],
                                              workspace=workspace)

    def walk(s):
        iva.paged_decode_attention_partial(s["q"], s["k_pool"], s["v_pool"], s["bt"], s["ctx"],
                                           partition_pages=pp, out=s["out"], workspace=workspace)

    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for s in sets:  # warm every code path before capture
            step(s)
            walk(s)
        torch.cuda.synchronize(dev)

        def make_graph(fn, reps):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for r in range(reps):
                    fn(sets[r % len(sets)])
            return g

        per_graph = len(sets) * max(1, 20 // len(sets))
        step_graph = None if args.eager else make_graph(step, per_graph)
        walk_graph = None if args.eager else make_graph(walk, per_graph)
        attn_graph = None if args.eager else make_graph(attention, per_graph)

        def run_steps(n):
            if step_graph is None:
                for i in range(n):
                    step(sets[i % len(sets)])
            else:
                for _ in range(n // per_graph):
                    step_graph.replay()
                for i in range(n % per_graph):
                    step(sets[i % len(sets)])

        run_steps(args.warmup)
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run_steps(args.steps)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        step_ms = e0.elapsed_time(e1) / args.steps

        def time_launches(graph, fn):
            """Average duration of fn's launches, back to back on the launch stream."""
            k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            if graph is not None:
                graph.replay()
                torch.cuda.synchronize(dev)
                reps = max(1, args.kernel_launches // per_graph)
                k0.record(stream)
                for _ in range(reps):
                    graph.replay()
                k1.record(stream)
                launches = reps * per_graph
            else:
                k0.record(stream)
                for i in range(args.kernel_launches):
                    fn(sets[i % len(sets)])
                k1.record(stream)
                launches = args.kernel_launches
            torch.cuda.synchronize(dev)
            return k0.elapsed_time(k1) * 1e3 / launches

        # dominant kernel alone: back-to-back launches of the paged walk
        walk_us = time_launches(walk_graph, walk)
        attn_us = time_launches(attn_graph, attention)

    return {"step_ms": step_ms, "walk_us": walk_us, "attn_us": attn_us,
            "pool_bytes": pool_bytes, "batch": batch}


def bench_ops(args, iva, torch, dev):
    """The hot path's data-movement kernels at realistic sizes (fp16, 8 kv heads, D 128),
    each as average time over back-to-back launches captured in one HIP graph: the append of
    16 x 512-token chunks (8192 rows; plain and with RoPE fused, into 16-bit and into FP8
    pages), the gather of the C2 batch into contiguous K/V (from 16-bit and from FP8
    pages), the kv_ops index gather /
    scatter kernels on a [32, 8, 4096, 128] cache, and the compaction's page moves (4096
    pages).  Every kernel's launches cycle through independent input and output sets
    (>= 512 MiB of distinct source bytes in all), so the 256 MiB MALL cannot serve a
    launch's reads from an earlier one.  Bytes are what each op must read and write; GB/s
    against the 8 TB/s HBM peak."""
    wl = iva.workloads
    hkv, d, es = 8, 128, 2
    gen = torch.Generator(device=dev).manual_seed(3)
    cpu_gen = torch.Generator().manual_seed(4)
    out = {}

    def timed(name, fn, nbytes, n_sets, reps=48, extra=None):
        # reps launches captured in one HIP graph, launch i on input set i % n_sets: the
        # replay times the device work, not the Python validation around each call
        for i in range(n_sets):
            fn(i)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(reps):
                fn(i % n_sets)
        graph.replay()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        del graph
        us = e0.elapsed_time(e1) * 1e3 / reps
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "bytes": int(nbytes), "gbps": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "input_sets": n_sets, **(extra or {})}

    # append: 8192 new rows per launch into a 64k-page pool (read the rows, write their
    # slots); 16 sets of rows, each into its own 512 pages
    n, n_app = 16 * 512, 16
    pages = 65536
    ks, vs = iva.pool_shapes(pages, hkv, d, 16, torch.float16)
    k_pool = torch.zeros(ks, dtype=torch.float16, device=dev)
    v_pool = torch.zeros(vs, dtype=torch.float16, device=dev)
    perm = torch.randperm(pages, generator=cpu_gen)
    rows = [(torch.randn(n, hkv, d, generator=gen, device=dev).half(),
             torch.randn(n, hkv, d, generator=gen, device=dev).half()) for _ in range(n_app)]
    slots = [(perm[i * (n // 16):(i + 1) * (n // 16)].repeat_interleave(16) * 16
              + torch.arange(n) % 16).int().to(dev) for i in range(n_app)]
    pos = (torch.arange(n) % 2048).int().to(dev)
    app_bytes = append_bytes(n, hkv, d, es)
    timed("append", lambda i: iva.kv_append(rows[i][0], rows[i][1], k_pool, v_pool, slots[i]),
          app_bytes, n_app)
    timed("append_rope", lambda i: iva.kv_append(rows[i][0], rows[i][1], k_pool, v_pool, slots[i],
                                                 rope_positions=pos), app_bytes + 4 * n, n_app)

    # the same rows as 16 chunks of 512 tokens that each start mid-page (offsets 1..15),
    # as chunked prefill after decode steps lands them (other pages than the above)
    def unaligned_slots(i):
        out, base = [], 8192 + i * 16 * 33
        for ch in range(16):
            o = 1 + (i * 16 + ch) % 15
            pg = perm[base + ch * 33: base + ch * 33 + 33]
            p = o + torch.arange(512)
            out.append(pg[p // 16] * 16 + p % 16)
        return torch.cat(out).int().to(dev)

    # a decode step's append (32 sequences, one row each at a random row of its own page)
    # and one 512-row chunk: the few-row launch shape (one kv head per lane)
    for name, nr in (("append_decode_step", 32), ("append_chunk512", 512)):
        sub = [(r[0][:nr].contiguous(), r[1][:nr].contiguous()) for r in rows]
        if nr == 32:
            sl = [(perm[20000 + 64 * i: 20000 + 64 * i + 32] * 16
                   + torch.randint(0, 16, (32,), generator=cpu_gen)).int().to(dev) for i in range(n_app)]
        else:
            sl = [s_[:nr] for s_ in slots]
        timed(name, lambda i, sub=sub, sl=sl: iva.kv_append(sub[i][0], sub[i][1], k_pool, v_pool, sl[i]),
              append_bytes(nr, hkv, d, es), n_app,
              extra={"rows": nr, "slots": "one row per sequence, each on its own page" if nr == 32
                     else "one page-aligned chunk"})
        del sub, sl

    slots_u = [unaligned_slots(i) for i in range(n_app)]
    timed("append_unaligned", lambda i: iva.kv_append(rows[i][0], rows[i][1], k_pool, v_pool,
                                                      slots_u[i]), app_bytes, n_app,
          extra={"slots": "16 chunks of 512 rows, each starting at page offset 1..15"})
    del slots_u
    # the same rows into FP8 pages (read fp16 rows, write codes and one factor per row)
    k8, v8 = (torch.zeros(shape, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
              for shape in iva.pool_shapes(pages, hkv, d, 16, torch.float8_e4m3fn))
    ks8, vs8 = (torch.ones(iva.scale_shape(pages, hkv), device=dev) for _ in range(2))
    app8_bytes = 2 * n * hkv * d * es + 2 * n * hkv * d + 2 * n * hkv * 4 + 4 * n
    timed("append_fp8", lambda i: iva.kv_append(rows[i][0], rows[i][1], k8, v8, slots[i],
                                                k_scale=ks8, v_scale=vs8), app8_bytes, n_app)
    timed("append_rope_fp8", lambda i: iva.kv_append(rows[i][0], rows[i][1], k8, v8, slots[i],
                                                     k_scale=ks8, v_scale=vs8,
                                                     rope_positions=pos),
          app8_bytes + 4 * n, n_app)
    del k8, v8, ks8, vs8, rows, slots
    # compaction's page moves: 4096 pages (K and V tiles of all kv heads) per launch to
    # free ids; 4 sets of source pages (every other page of 8192) and destinations
    n_mv = 4
    src = [torch.arange(8192 * i, 8192 * (i + 1), 2, dtype=torch.int32, device=dev)
           for i in range(n_mv)]
    dst = [torch.arange(40960 + 4096 * i, 40960 + 4096 * (i + 1), dtype=torch.int32, device=dev)
           for i in range(n_mv)]
    timed("copy_pages", lambda i: iva.copy_pages(k_pool, v_pool, src[i], dst[i]),
          2 * 4096 * 2 * hkv * 16 * d * es + 8 * 4096, n_mv)
    # the same page moves at the chunk append's size (512 pages: the bytes an 8192-row
    # append reads and writes), 16 sets: what a plain copy of that size reaches, start-up
    # and tail included
    src = [torch.arange(1024 * i, 1024 * (i + 1), 2, dtype=torch.int32, device=dev)
           for i in range(16)]
    dst = [torch.arange(40960 + 512 * i, 40960 + 512 * (i + 1), dtype=torch.int32, device=dev)
           for i in range(16)]
    timed("copy_pages_512", lambda i: iva.copy_pages(k_pool, v_pool, src[i], dst[i]),
          2 * 512 * 2 * hkv * 16 * d * es + 8 * 512, 16,
          extra={"pages": 512, "note": "the bytes of the 8192-row append"})
    del k_pool, v_pool
    # gather of the C2 batch into contiguous [B, Hkv, max L, D]: 4 batches (pools and
    # outputs)
    lengths = wl.c2_lengths(seed=0)
    lmax = max(lengths)
    n_ga = 4
    gsets = []
    for i in range(n_ga):
        dd = wl.decode_batch(lengths, 32, hkv, d, torch.float16, seed=100 + i, device=dev)
        lay = dd["layout"]
        kg = torch.empty(len(lengths), hkv, lmax, d, dtype=torch.float16, device=dev)
        gsets.append((dd["k_pool"], dd["v_pool"], lay.block_tables.to(dev),
                      lay.context_lens.to(dev), kg, torch.empty_like(kg)))
    timed("gather", lambda i: iva.kv_gather(gsets[i][0], gsets[i][1], gsets[i][2], gsets[i][3],
                                            out_len=lmax, out=(gsets[i][4], gsets[i][5])),
          2 * sum(lengths) * hkv * d * es + 2 * gsets[0][4].numel() * es, n_ga)
    # the same batch from FP8 pages (codes and factors of each attended row read,
    # dequantized into fp16 outputs)
    f8sets = []
    for i in range(n_ga):
        k_p, v_p, bt_, ctx_, kg, vg = gsets[i]
        f8 = [torch.randint(0, 256, s_, dtype=torch.uint8, generator=gen, device=dev)
              .view(torch.float8_e4m3fn) for s_ in iva.pool_shapes(k_p.shape[0], hkv, d, 16,
                                                                   torch.float8_e4m3fn)]
        sc = [torch.rand(iva.scale_shape(k_p.shape[0], hkv), generator=gen, device=dev) + 0.5
              for _ in range(2)]
        f8sets.append((f8[0], f8[1], sc[0], sc[1], bt_, ctx_, kg, vg))
    del gsets
    timed("gather_fp8", lambda i: iva.kv_gather(
        f8sets[i][0], f8sets[i][1], f8sets[i][4], f8sets[i][5], out_len=lmax,
        out=(f8sets[i][6], f8sets[i][7]), k_scale=f8sets[i][2], v_scale=f8sets[i][3]),
        2 * sum(lengths) * hkv * (d + 4) + 2 * f8sets[0][6].numel() * es, n_ga,
        extra={"pages": "fp8", "out_dtype": "f16"})
    del f8sets
    # kv_ops' index kernels on a contiguous cache: gather 1024 positions, scatter 1024
    # rows, through the C ABI on preallocated buffers (kv_ops itself checks the indices
    # on the host, a synchronisation per call, and its scatter copies the whole cache
    # first, a torch copy); 4 caches, index sets and dense buffers
    n_ix = 4
    caches = [torch.randn(32, hkv, 4096, d, generator=gen, device=dev).half() for _ in range(n_ix)]
    idxs = [torch.randperm(4096, generator=cpu_gen)[:1024].to(dev) for _ in range(n_ix)]
    dense = [torch.randn(32, hkv, 1024, d, generator=gen, device=dev).half() for _ in range(n_ix)]
    code = iva.dtype_code(torch.float16)
    row_bytes = 32 * hkv * 1024 * d * es

    def stream():
        return torch.cuda.current_stream(dev).cuda_stream

    timed("index_gather", lambda i: iva._abi.call(
        "ivakv_index_gather", caches[i].data_ptr(), *caches[i].stride(), idxs[i].data_ptr(), 1024,
        32, hkv, 4096, d, dense[i].data_ptr(), code, stream()), 2 * row_bytes + 8 * 1024, n_ix)
    timed("index_scatter", lambda i: iva._abi.call(
        "ivakv_index_scatter", caches[i].data_ptr(), *caches[i].stride(), idxs[i].data_ptr(), 1024,
        dense[i].data_ptr(), *dense[i].stride(), 32, hkv, 4096, d, code, stream()),
        2 * row_bytes + 8 * 1024, n_ix)
    return {"metric": "hot-path data-movement kernels GB/s (fraction of 8 TB/s HBM)",
            "workload": "ops", "dtype": "f16", "data": "synthetic",
            "config": {"num_kv_heads": hkv, "head_dim": d, "block_size": 16,
                       "launch": "hip graph of back-to-back launches over rotated input sets"},
            "kernels": out}


def main():
    args = parse_args()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc, context=args.context, rdreq_dir=args.rdreq_dir)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(sharding the path over several GPUs is not built)"}))
        sys.exit(2)

    import torch
    import __graft_entry__

    iva = __graft_entry__.load_package()
    iva._abi.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = iva.workloads
    if args.workload != "c2":
        fn = {"c3": bench_c3, "c4": bench_c4, "c5": bench_c5, "prefill": bench_prefill,
              "c2fp8": bench_c2fp8, "ops": bench_ops, "ceiling": bench_ceiling}[args.workload]
        print(json.dumps(fn(args, iva, torch, dev)), flush=True)
        return

    hq, hkv, d, esize = 32, 8, 128, 2
    lengths = wl.c2_lengths(seed=0)
    context_desc = "U[512,4096] seed 0"
    if args.context != "c2":
        lengths = [int(args.context)] * len(lengths)
        context_desc = f"{int(args.context)} (every sequence)"
    m = measure_decode(args, iva, torch, dev, lengths)
    step_ms, walk_us, attn_us, pool_bytes, batch = (
        m["step_ms"], m["walk_us"], m["attn_us"], m["pool_bytes"], m["batch"])
    target = None
    if (args.context == "c2" and args.target_4k and not args.partition_pages
            and not args.eager and not args.copy_calibration):
        # the north-star target's own shape: every sequence at context 4096, on pools
        # allocated afresh (the C2 pools' cached blocks returned to the device first)
        torch.cuda.empty_cache()
        t_len = [4096] * batch
        mt = measure_decode(args, iva, torch, dev, t_len)
        t_append, t_attn = algorithmic_bytes(t_len, 32, 8, 128, 2)
        t_ach = t_attn / (mt["walk_us"] * 1e-6) / 1e9
        target = {"context": 4096, "batch": batch, "kernel_us": round(mt["walk_us"], 3),
                  "achieved": round(t_ach, 1), "frac": round(t_ach / HBM_PEAK_GBS, 4),
                  "frac_of_measured_read_reference": None,
                  "algorithmic_bytes": t_attn, "attention_us": round(mt["attn_us"], 3),
                  "step_us": round(mt["step_ms"] * 1e3, 3),
                  "step_gbs": round((t_append + t_attn) / (mt["step_ms"] * 1e-3) / 1e9, 1),
                  "traffic": read_traffic("4096"),
                  "traffic_source": "profiles/decode_attn_ctx4096_traffic.json (committed "
                                    "counter runs; not measured in this run)"}
    if args.copy_calibration:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(7)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize(dev)

    ceiling = None
    if not args.copy_calibration and not args.eager:
        torch.cuda.empty_cache()
        ceiling = measure_ceiling(torch, dev)

    append_b, attn_b = algorithmic_bytes(lengths, hq, hkv, d, esize)
    step_s = step_ms * 1e-3
    value = (append_b + attn_b) / step_s / 1e9
    achieved = attn_b / (walk_us * 1e-6) / 1e9

    traffic = read_traffic(args.context)

    cpu = None
    if args.cpu_reps > 0:
        t_cpu, threads = cpu_baseline(lengths, hq, hkv, d, args.cpu_reps)
        cpu = {"value": round((append_b + attn_b) / t_cpu / 1e9, 3), "unit": "GB/s",
               "cores": threads, "kind": "port",
               "sample": (f"full C2 batch ({batch} seqs), one decode step of the reference torch "
                          f"path restated on CPU in fp32 (torch.cat append + AttentionTorch math), "
                          f"median of {args.cpu_reps} reps after 3 warm-ups, "
                          f"{t_cpu * 1e3:.1f} ms/step, {cpu_model()}"),
               "ms_per_step": round(t_cpu * 1e3, 2)}

    walk_name = (f"{WALK_KERNEL}<f16,128>" if not args.partition_pages
                 else "decode_partial_kernel<f16,128>")
    if target is not None and ceiling is not None:
        target["frac_of_measured_read_reference"] = round(
            target["achieved"] / ceiling["read_reference_gbs"], 4)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "C2 paged decode attention + 1-row KV append per sequence",
                   "batch": batch, "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d,
                   "block_size": 16, "context": context_desc,
                   "mean_context": round(sum(lengths) / batch, 1), "pools_rotated": args.pools,
                   "pool_bytes_total": pool_bytes, "launch": "eager" if args.eager else "hip graph",
                   "walk": "partitioned, %d pages" % args.partition_pages
                   if args.partition_pages else "stream",
                   "step_ops": "ivakv_append + ivakv_decode_attn" if args.unfused or
                   args.partition_pages else "ivakv_decode_append_attn (fused)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": (f"profiles/{traffic_path(args.context).name}: committed "
                                        "rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this walk, "
                                        "scaled by a plain copy; not measured in this run")
                     if traffic is not None else None,
                     "kernel": walk_name,
                     "kernel_us": round(walk_us, 3), "algorithmic_bytes": attn_b,
                     "frac_of_measured_read_reference":
                         round(achieved / ceiling["read_reference_gbs"], 4) if ceiling else None},
        "ceiling": ceiling,
        "cpu_baseline": cpu,
        "tokens_per_s": round(batch / step_s, 1),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "attention_us": round(attn_us, 3),
        "step_bytes": {"append": append_b, "attention": attn_b},
        "target_4k": target,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
