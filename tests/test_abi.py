"""The C ABI without a GPU: the library loads, exports exactly what include/ivakv.h
declares, and rejects bad arguments on the host before any launch."""
from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ivakv.h"
FAKE = 0x10000  # a 16-byte-aligned non-null address; never dereferenced by these calls


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ivakv_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree(iva):
    names = declared_symbols()
    assert len(names) >= 10
    assert names == sorted(iva._abi.SIGNATURES)


def test_library_exports_every_declared_symbol(iva):
    lib = iva._abi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} not exported by libivakv.so"
    assert lib.ivakv_abi_version() == iva._abi.ABI_VERSION == 2


def call(iva, name, *args):
    return getattr(iva._abi.lib(), name)(*args)


def test_append_argument_checks(iva):
    a = iva._abi
    ok_args = [FAKE, FAKE, 512, 64, 512, 64, FAKE, FAKE, FAKE, 3, 8, 64, 16, 4]
    assert call(iva, "ivakv_append", *ok_args[:13], 4, 9, None) == a.E_DTYPE
    assert "dtype" in a.last_error()
    assert call(iva, "ivakv_append", FAKE, FAKE, 512, 64, 512, 64, FAKE, FAKE, FAKE,
                3, 8, 60, 16, 4, a.F16, None) == a.E_SHAPE
    assert call(iva, "ivakv_append", None, FAKE, 512, 64, 512, 64, FAKE, FAKE, FAKE,
                3, 8, 64, 16, 4, a.F16, None) == a.E_ARG
    assert call(iva, "ivakv_append", FAKE, FAKE, -1, 64, 512, 64, FAKE, FAKE, FAKE,
                3, 8, 64, 16, 4, a.F16, None) == a.E_ARG
    assert call(iva, "ivakv_append", FAKE, FAKE, 512, 64, 512, 64, FAKE, FAKE, FAKE,
                -3, 8, 64, 16, 4, a.F16, None) == a.E_ARG
    # zero tokens is a no-op that succeeds without touching the device
    assert call(iva, "ivakv_append", None, None, 0, 0, 0, 0, None, None, None,
                0, 8, 64, 16, 4, a.F16, None) == a.OK


def test_gather_argument_checks(iva):
    a = iva._abi
    assert call(iva, "ivakv_gather", FAKE, FAKE, FAKE, FAKE, 2, 4, 8, 64, 16, 8, 64,
                FAKE, FAKE, 5, None) == a.E_DTYPE
    assert call(iva, "ivakv_gather", FAKE, FAKE, FAKE, FAKE, 2, 4, 8, 63, 16, 8, 64,
                FAKE, FAKE, a.F32, None) == a.E_SHAPE
    assert call(iva, "ivakv_gather", FAKE, FAKE, None, FAKE, 2, 4, 8, 64, 16, 8, 64,
                FAKE, FAKE, a.F32, None) == a.E_ARG
    assert call(iva, "ivakv_gather", FAKE + 4, FAKE, FAKE, FAKE, 2, 4, 8, 64, 16, 8, 64,
                FAKE, FAKE, a.F32, None) == a.E_ARG
    assert "aligned" in a.last_error()
    assert call(iva, "ivakv_gather", None, None, None, None, 0, 4, 8, 64, 16, 8, 64,
                None, None, a.F32, None) == a.OK


def decode_args(iva, **over):
    a = iva._abi
    args = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, ctx=FAKE, out=FAKE, ws=None, ws_bytes=0,
                batch=4, hq=32, hkv=8, d=128, bs=16, max_blocks=256, num_pages=1000,
                scale=0.088, window=0, n_sink=0, pp=0, dtype=a.F16, stream=None)
    args.update(over)
    return list(args.values())


def test_decode_argument_checks(iva):
    a = iva._abi
    name = "ivakv_decode_attn"
    assert call(iva, name, *decode_args(iva, dtype=3)) == a.E_DTYPE
    assert call(iva, name, *decode_args(iva, bs=32)) == a.E_SHAPE
    assert call(iva, name, *decode_args(iva, d=96)) == a.E_SHAPE
    assert call(iva, name, *decode_args(iva, hq=34)) == a.E_SHAPE
    assert call(iva, name, *decode_args(iva, hq=8 * 17)) == a.E_SHAPE
    assert call(iva, name, *decode_args(iva, q=None)) == a.E_ARG
    assert call(iva, name, *decode_args(iva, num_pages=0)) == a.E_ARG
    assert call(iva, name, *decode_args(iva, n_sink=-1)) == a.E_ARG
    # 256 blocks / 16 pages per partition -> split-K needs a workspace
    assert call(iva, name, *decode_args(iva)) == a.E_WORKSPACE
    assert "workspace" in a.last_error()
    assert call(iva, name, *decode_args(iva, ws=FAKE, ws_bytes=100)) == a.E_WORKSPACE
    assert call(iva, name, *decode_args(iva, batch=0)) == a.OK
    for entry in ("ivakv_decode_attn_partial", "ivakv_decode_attn_merge"):
        assert call(iva, entry, *decode_args(iva, bs=8)) == a.E_SHAPE


def test_workspace_size(iva):
    ws = iva.decode_workspace_bytes
    # explicit partitions, one per sequence: no workspace
    assert ws(32, 32, 8, 128, 16, 16, partition_pages=16) == 0
    # explicit partitions: 256 blocks / 16 = 16 partitions of G=4 heads x (128 + 2) fp32
    assert ws(32, 32, 8, 128, 16, 256, partition_pages=16) == 32 * 8 * 16 * 4 * 130 * 4
    # a window bounds the partitions: 4 sinks + 4096 window -> 1 + 256 + 1 pages
    assert ws(4, 32, 8, 128, 16, 8192, window=4096, n_sink=4, partition_pages=16) == \
        4 * 8 * 17 * 4 * 130 * 4
    # default (stream walk): one slot per wave of the wave budget plus one per
    # (sequence, kv head), then the batch's page prefix (B + 1 ints, padded to 4)
    stream = (4096 + 32 * 8) * 4 * 130 * 4 + 36 * 4
    assert ws(32, 32, 8, 128, 16, 256) == stream
    assert ws(32, 32, 8, 128, 16, 16) == stream
    with pytest.raises(iva._abi.IvakvError):
        ws(1, 3, 2, 128, 16, 4)


def test_ops_refuse_cpu_tensors(iva):
    kp = torch.zeros(iva.pool_shapes(4, 2, 64, 16, torch.float16)[0], dtype=torch.float16)
    vp = torch.zeros(iva.pool_shapes(4, 2, 64, 16, torch.float16)[1], dtype=torch.float16)
    rows = torch.zeros(1, 2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        iva.kv_append(rows, rows, kp, vp, torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        iva.paged_decode_attention(torch.zeros(1, 4, 64, dtype=torch.float16), kp, vp,
                                   torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))


def test_kv_ops_errors_match_reference(iva):
    """kv_ops raises the reference's ValueErrors (kv_ops_triton.py:126-127,142-143)."""
    kv = torch.zeros(1, 1, 4, 8)
    with pytest.raises(ValueError, match="Values tensor required"):
        iva.kv_ops(kv, torch.tensor([0]), None, "scatter")
    with pytest.raises(ValueError, match="Unknown operation"):
        iva.kv_ops(kv, torch.tensor([0]), None, "compact")


def test_pool_shapes(iva):
    assert iva.pool_shapes(10, 8, 128, 16, torch.float16) == ((10, 8, 16, 16, 8), (10, 8, 128, 16))
    assert iva.pool_shapes(10, 8, 64, 16, torch.float32) == ((10, 8, 16, 16, 4), (10, 8, 64, 16))
    with pytest.raises(ValueError):
        iva.pool_shapes(1, 1, 12, 16, torch.bfloat16)


def test_fp8_entry_argument_checks(iva):
    """Host-side validation of the FP8 prefill and fused decode entry points (nothing is
    launched: every call fails before a kernel would start)."""
    a = iva._abi

    def prefill8(**over):
        args = dict(q=FAKE, k=FAKE, v=FAKE, ks=FAKE, vs=FAKE, bt=FAKE, ctx=FAKE, qs=FAKE,
                    n_tok=8, out=FAKE, batch=2, hq=8, hkv=2, d=128, bs=16, max_blocks=8,
                    num_pages=16, max_q=4, scale=0.088, window=0, n_sink=0, dtype=a.F16,
                    stream=None)
        args.update(over)
        return call(iva, "ivakv_prefill_attn_fp8", *args.values())

    assert prefill8(dtype=a.F32) == a.E_DTYPE
    assert "fp16 or bf16" in a.last_error()
    assert prefill8(ks=None) == a.E_ARG
    assert prefill8(vs=FAKE + 4) == a.E_ARG       # factors must be 16-byte aligned
    assert prefill8(d=96) == a.E_SHAPE
    assert prefill8(hq=9) == a.E_SHAPE
    assert prefill8(n_tok=-1) == a.E_ARG
    assert prefill8(max_q=0) == a.OK              # nothing to do
    assert prefill8(n_tok=0) == a.OK

    def fused8(**over):
        args = dict(q=FAKE, kn=FAKE, vn=FAKE, k=FAKE, v=FAKE, ks=FAKE, vs=FAKE, bt=FAKE,
                    ctx=FAKE, out=FAKE, ws=None, ws_bytes=0, batch=2, hq=8, hkv=2, d=128,
                    bs=16, max_blocks=8, num_pages=16, scale=0.088, window=0, n_sink=0,
                    dtype=a.F16, stream=None)
        args.update(over)
        return call(iva, "ivakv_decode_append_attn_fp8", *args.values())

    assert fused8(dtype=a.F32) == a.E_DTYPE
    assert fused8(ks=None) == a.E_ARG
    assert fused8(kn=None) == a.E_ARG
    assert fused8() == a.E_WORKSPACE              # the stream walk needs a workspace
    assert fused8(bs=8) == a.E_SHAPE


def test_prefill_and_copy_pages_argument_checks(iva):
    """ivakv_prefill_attn takes the row count of q / out (query_start is bounded by it in
    the kernel); ivakv_copy_pages takes the pool's page count (moves outside it are
    skipped in the kernel)."""
    a = iva._abi

    def prefill(**over):
        args = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, ctx=FAKE, qs=FAKE, n_tok=8, out=FAKE,
                    batch=2, hq=8, hkv=2, d=128, bs=16, max_blocks=8, num_pages=16, max_q=4,
                    scale=0.088, window=0, n_sink=0, dtype=a.F16, stream=None)
        args.update(over)
        return call(iva, "ivakv_prefill_attn", *args.values())

    assert prefill(n_tok=-1) == a.E_ARG
    assert "n_tok" in a.last_error()
    assert prefill(d=96) == a.E_SHAPE
    assert prefill(n_tok=0) == a.OK
    assert prefill(batch=0) == a.OK

    def copy(**over):
        args = dict(k=FAKE, v=FAKE, ks=None, vs=None, src=FAKE, dst=FAKE, n=4, pages=16,
                    hkv=8, d=128, bs=16, eb=2, stream=None)
        args.update(over)
        return call(iva, "ivakv_copy_pages", *args.values())

    assert copy(pages=-1) == a.E_ARG
    assert "pages=-1" in a.last_error()
    assert copy(eb=3) == a.E_ARG
    assert copy(ks=FAKE) == a.E_ARG               # both factor tensors or neither
    assert copy(n=0) == a.OK


def test_error_messages_are_per_thread(iva):
    """ivakv_last_error is thread-local: two threads failing different entry points at
    the same time each read back their own message after every call."""
    import threading

    a = iva._abi
    start = threading.Barrier(2)
    bad = []

    def fail_append():
        start.wait()
        for _ in range(3000):
            st = call(iva, "ivakv_append", FAKE, FAKE, 512, 64, 512, 64, FAKE, FAKE, FAKE,
                      3, 8, 64, 16, 4, 9, None)
            msg = a.last_error()
            if st != a.E_DTYPE or not msg.startswith("ivakv_append"):
                bad.append(("append", st, msg))

    def fail_gather():
        start.wait()
        for _ in range(3000):
            st = call(iva, "ivakv_gather", FAKE, FAKE, FAKE, FAKE, 2, 4, 8, 63, 16, 8, 64,
                      FAKE, FAKE, a.F16, None)
            msg = a.last_error()
            if st == a.OK or not msg.startswith("ivakv_gather"):
                bad.append(("gather", st, msg))

    threads = [threading.Thread(target=f) for f in (fail_append, fail_gather)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not bad, bad[:3]
