"""Writes the committed golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference publishes no vectors for this path (it has no tests), so the
fixtures are produced here on the CPU:
  c1.json            seed and SHA-256 digests of config C1 (fp32 append of
                     4 sequences {17, 64, 129, 200} x 8 heads x 64, block 16,
                     then gather): the inputs drawn from the seed and the
                     gathered K/V computed by the numpy oracle.
  decode_tiny.npz    a tiny decode-attention case (2 sequences, GQA 4/2,
                     head_dim 8, window 5 + 2 sinks) whose expected output is
                     evaluated term by term in pure Python
                     (oracle.paged_kv.decode_attention_loops), independently
                     of the vectorised oracle and of the kernels.
"""
from __future__ import annotations

import hashlib
import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402
from oracle import paged_kv as orc  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def make_c1(seed: int = 0) -> dict:
    iva = __graft_entry__.load_package()
    w = iva.workloads.c1_append_gather(seed=seed)
    lay = w["layout"]
    k_new = w["k_new"].numpy().view(np.uint32)
    v_new = w["v_new"].numpy().view(np.uint32)
    kp, vp = orc.empty_pools(w["num_pages"], 8, 64, 16, np.uint32)
    orc.append(kp, vp, k_new, v_new, w["slot_mapping"].numpy())
    ko, vo = orc.gather(kp, vp, lay.block_tables.numpy(), lay.context_lens.numpy())
    return {
        "config": "C1: fp32 append+gather, lengths {17,64,129,200}, Hkv 8, D 64, block 16, 64-page pool",
        "seed": seed,
        "k_new_sha256": sha(k_new),
        "v_new_sha256": sha(v_new),
        "block_tables": lay.block_tables.tolist(),
        "k_out_sha256": sha(ko),
        "v_out_sha256": sha(vo),
    }


def make_decode_tiny(seed: int = 0) -> dict:
    rng = np.random.default_rng(seed)
    lengths = [37, 9]
    hq, hkv, d, bs = 4, 2, 8, 16
    window, n_sink = 5, 2
    num_pages = 6
    bt = np.array([[4, 0, 2], [5, -1, -1]], dtype=np.int32)
    q = rng.standard_normal((2, hq, d)).astype(np.float32)
    kp, vp = orc.empty_pools(num_pages, hkv, d, bs, np.float32)
    rows_k, rows_v = [], []
    for b, n in enumerate(lengths):
        k = rng.standard_normal((n, hkv, d)).astype(np.float32)
        v = rng.standard_normal((n, hkv, d)).astype(np.float32)
        slots = np.array([bt[b, p // bs] * bs + p % bs for p in range(n)])
        orc.append(kp, vp, k, v, slots)
        rows_k.append(k.transpose(1, 0, 2))
        rows_v.append(v.transpose(1, 0, 2))
    expected = orc.decode_attention_loops(q.tolist(), [r.tolist() for r in rows_k],
                                          [r.tolist() for r in rows_v], lengths,
                                          1 / math.sqrt(d), window, n_sink)
    return dict(q=q, k_pool=kp, v_pool=vp, block_tables=bt, context_lens=np.array(lengths, np.int32),
                window=np.int32(window), n_sink=np.int32(n_sink), expected=np.array(expected))


if __name__ == "__main__":
    (HERE / "c1.json").write_text(json.dumps(make_c1(), indent=1) + "\n")
    np.savez(HERE / "decode_tiny.npz", **make_decode_tiny())
    print("wrote", HERE / "c1.json", HERE / "decode_tiny.npz")
