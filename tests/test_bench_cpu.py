"""bench.py on the CPU: the contract's refusal of more than one GPU, the algorithmic bytes
the C2 line and its profiles are quoted on, and the HBM-traffic summary's arithmetic
(copy-calibrated FETCH_SIZE / WRITE_SIZE, and the read bytes counted by request size)
on synthetic rocprofv3 counter files."""
from __future__ import annotations

import csv
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import bench  # noqa: E402  (no GPU work at import)

WALK = "void ivakv::(anonymous namespace)::decode_stream_kernel<ivakv::(anonymous namespace)::TileOps<1, 128> >(x)"
COPY = "void at::native::vectorized_elementwise_kernel<4, at::native::copy_kernel>(x)"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_c2_algorithmic_bytes(iva):
    """The walk's bytes in the C2 line, its roofline and its profiles: K + V of every
    attended row, q and out, one 4-byte block-table entry per page, the context lengths."""
    lengths = iva.workloads.c2_lengths(seed=0)
    append, attn = bench.algorithmic_bytes(lengths, 32, 8, 128, 2)
    assert attn == 287_114_504
    # the append's one formula: K and V rows read and written, plus the slot map
    assert append == bench.append_bytes(32, 8, 128, 2) == 4 * 32 * 8 * 128 * 2 + 4 * 32
    # every sequence at 4096 (the target_4k figure)
    assert bench.algorithmic_bytes([4096] * 32, 32, 8, 128, 2)[1] == 537_428_096


def _write_counters(directory: Path, rows):
    directory.mkdir(parents=True)
    with (directory / "run_counter_collection.csv").open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for k, c, v in rows:
            w.writerow({"Kernel_Name": k, "Counter_Name": c, "Counter_Value": v})


def test_traffic_summary_scales_and_cross_checks(tmp_path, monkeypatch):
    copy_kib = bench.COPY_BYTES / 1024
    walk_read = 288_000_000                       # bytes the synthetic walk reads
    fetch = [(WALK, "FETCH_SIZE", walk_read / 2 / 1024)] * 3 + \
            [(COPY, "FETCH_SIZE", copy_kib / 2)] * 10          # the counter reads half
    write = [(WALK, "WRITE_SIZE", 2500.0)] * 3 + [(COPY, "WRITE_SIZE", copy_kib)] * 10
    n128 = walk_read // 128
    rdreq = []
    for k, n in ((WALK, n128), (COPY, bench.COPY_BYTES // 128)):
        rdreq += [(k, "TCC_EA0_RDREQ_sum", n), (k, "TCC_EA0_RDREQ_32B_sum", 0),
                  (k, "TCC_EA0_RDREQ_64B_sum", 0), (k, "TCC_EA0_RDREQ_128B_sum", n)]
    _write_counters(tmp_path / "f", fetch)
    _write_counters(tmp_path / "w", write)
    _write_counters(tmp_path / "r", rdreq)
    out = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "traffic_path", lambda context: out)
    bench.summarize_pmc(str(tmp_path / "f"), str(tmp_path / "w"), rdreq_dir=str(tmp_path / "r"))
    s = json.loads(out.read_text())
    assert s["fetch_scale"] == 2.0 and s["write_scale"] == 1.0
    assert s["hbm_read_bytes_per_launch"] == walk_read
    assert s["hbm_write_bytes_per_launch"] == 2500 * 1024
    assert s["rdreq_read_bytes_per_launch"] == n128 * 128
    assert s["rdreq_copy_read_bytes"] == bench.COPY_BYTES
    assert abs(s["rdreq_over_scaled_fetch"] - n128 * 128 / walk_read) < 1e-4


def test_committed_traffic_summary_is_read():
    assert bench.read_traffic("c2") == json.loads(
        (ROOT / "profiles" / "decode_attn_c2_traffic.json").read_text())["hbm_bytes_per_launch"]


def test_prefill_split_default(iva):
    """The split-prefill default on the shapes the measurements were taken on."""
    from importlib import import_module
    ops = import_module("iva_amd.ops")
    split = ops.prefill_split_default
    # C3's prefill layer: 16 x 512 rows, 16 heads, a 48-page table -> single launch
    assert not split(16, 16, 16, 16 * 512, 512, 48, 16)
    # short batches (4 x 128 at 256 keys, 8 x 64 at 1024 keys) -> single launch
    assert not split(4, 32, 8, 4 * 128, 128, 16, 16)
    assert not split(8, 32, 8, 8 * 64, 64, 64, 16)
    # the prefill line: 16 x 512 rows, 32 heads, 2048 keys: work bound 2^29 -> split
    assert split(16, 32, 8, 16 * 512, 512, 128, 16)
    # a table wider than 4096 keys (C5's pools, long prompts) -> split, even for one row
    assert split(1, 32, 8, 1, 1, 1024, 16)
    # ... unless a window bounds the walk: 256 + 64 + 4 keys
    assert not split(1, 32, 8, 64, 64, 1024, 16, window=256, n_sink=4)
    # few row blocks on a long walk (one sequence, 128 rows at 4096 keys; 16 rows at 2048
    # keys; four sequences of 128 rows at 2048 keys) -> split; at 1024 keys -> single launch
    assert split(1, 32, 8, 128, 128, 256, 16)
    assert split(1, 32, 8, 16, 16, 128, 16)
    assert split(4, 32, 8, 4 * 128, 128, 128, 16)
    assert not split(1, 32, 8, 16, 16, 64, 16)
    assert not split(16, 32, 8, 16 * 64, 64, 64, 16)
    # ... and with 256 row-block workgroups (four 512-row chunks at 2048 keys) -> single
    assert not split(4, 32, 8, 4 * 512, 512, 128, 16)
    # outside the split path's limits -> single launch
    assert not split(ops.SPLIT_MAX_BATCH + 1, 32, 8, 4096, 512, 1024, 16)
    assert not split(4, 32768, 32768, 4, 1, 1024, 16)
