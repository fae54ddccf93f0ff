"""ivakv_decode_append_attn_noalloc (the fused decode step with its workspace in the
library's static scratch) against ivakv_decode_append_attn with a caller workspace,
through the C ABI: identical outputs and identical pools (bit for bit: same plan, same
kernels), on calls in a row with shrinking inputs (the scratch keeps the previous
call's contents), on the stream walk and on the one-partition path; a geometry whose
workspace exceeds the scratch is refused before any launch; the scratch is mapped on a
device by the first noalloc call there, not by the rest of the library."""
from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _step_inputs(iva, lengths, hq, hkv, d, dtype, seed, dev):
    w = iva.workloads.decode_batch(lengths, hq, hkv, d, dtype, seed=seed, device=dev,
                                   scale=1 / math.sqrt(d))
    gen = torch.Generator(device=dev).manual_seed(seed + 7)
    k_new = (torch.randn(len(lengths), hkv, d, generator=gen, device=dev) / math.sqrt(d)).to(dtype)
    v_new = (torch.randn(len(lengths), hkv, d, generator=gen, device=dev) / math.sqrt(d)).to(dtype)
    lay = w["layout"]
    return w, k_new, v_new, lay.block_tables.to(dev), lay.context_lens.to(dev)


def _run(iva, entry, w, k_new, v_new, bt, ctx, window, n_sink, dev):
    """One fused step on copies of the pools; returns (out, k_pool, v_pool)."""
    q = w["q"]
    kp, vp = w["k_pool"].clone(), w["v_pool"].clone()
    out = torch.full_like(q, float("nan"))
    b, hq, d = q.shape
    hkv = kp.shape[1]
    code = iva.dtype_code(q.dtype)
    stream = torch.cuda.current_stream(dev).cuda_stream
    common = (b, hq, hkv, d, 16, bt.shape[1], kp.shape[0], 1 / math.sqrt(d), window, n_sink,
              code, stream)
    if entry == "ivakv_decode_append_attn":
        nbytes = iva.decode_workspace_bytes(b, hq, hkv, d, 16, bt.shape[1], window, n_sink)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        iva._abi.call(entry, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), kp.data_ptr(),
                      vp.data_ptr(), bt.data_ptr(), ctx.data_ptr(), out.data_ptr(),
                      ws.data_ptr(), ws.numel(), *common)
    else:
        iva._abi.call(entry, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), kp.data_ptr(),
                      vp.data_ptr(), bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), *common)
    torch.cuda.synchronize(dev)
    return out, kp, vp


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


CALLS = [
    # (lengths, hq, hkv, d, dtype, window, n_sink): stream walk at C2's shape, then a
    # smaller stream-walk batch, then a one-partition batch (a unit per CU, short tables)
    ("c2", None, 32, 8, 128, torch.float16, 0, 0),
    ("small", [700, 33, 1, 2049, 160], 32, 8, 128, torch.float16, 512, 4),
    ("one_partition", [300] * 40, 16, 16, 64, torch.bfloat16, 0, 0),
]


def test_scratch_is_mapped_by_the_first_noalloc_call(iva, dev):
    """The 64 MiB scratch sits in a code object of its own: the workspace entry point and
    the rest of the library leave it unmapped, the first noalloc call on the device maps
    it (device free memory drops by at least 64 MiB then, and not before).  This file is
    the only caller of the noalloc entry, and this test its first call in the process."""
    lengths = [700, 1500, 33]
    w, kn, vn, bt, ctx = _step_inputs(iva, lengths, 32, 8, 128, torch.float16, 31, dev)
    _run(iva, "ivakv_decode_append_attn", w, kn, vn, bt, ctx, 0, 0, dev)
    torch.cuda.synchronize(dev)
    free0 = torch.cuda.mem_get_info(dev)[0]
    _run(iva, "ivakv_decode_append_attn", w, kn, vn, bt, ctx, 0, 0, dev)
    free1 = torch.cuda.mem_get_info(dev)[0]
    _run(iva, "ivakv_decode_append_attn_noalloc", w, kn, vn, bt, ctx, 0, 0, dev)
    free2 = torch.cuda.mem_get_info(dev)[0]
    mib = 1 << 20
    print(f"device free memory: {free0 / mib:.0f} MiB, after a workspace call "
          f"{free1 / mib:.0f}, after the first noalloc call {free2 / mib:.0f}", flush=True)
    assert free0 - free1 < 64 * mib
    assert free1 - free2 >= 64 * mib


def test_noalloc_matches_the_workspace_entry(iva, dev):
    for i, (name, lengths, hq, hkv, d, dtype, window, n_sink) in enumerate(CALLS):
        if lengths is None:
            lengths = iva.workloads.c2_lengths(seed=0)
        print(f"noalloc call {i}: {name} B={len(lengths)} Hq={hq} Hkv={hkv} D={d}", flush=True)
        w, kn, vn, bt, ctx = _step_inputs(iva, lengths, hq, hkv, d, dtype, 40 + i, dev)
        o1, k1, v1 = _run(iva, "ivakv_decode_append_attn", w, kn, vn, bt, ctx, window, n_sink, dev)
        o2, k2, v2 = _run(iva, "ivakv_decode_append_attn_noalloc", w, kn, vn, bt, ctx, window,
                          n_sink, dev)
        assert not torch.isnan(o1).any()
        assert torch.equal(_bits(o1), _bits(o2)), name
        assert torch.equal(_bits(k1), _bits(k2)) and torch.equal(_bits(v1), _bits(v2)), name


def test_noalloc_refuses_a_workspace_beyond_the_scratch(iva, dev):
    a = iva._abi
    # 8192 sequences x 8 kv heads at GQA 4, D 128: (4096 + 65536) slots x 2080 B > 64 MiB
    assert iva.decode_workspace_bytes(8192, 32, 8, 128, 16, 256) > 64 << 20
    # null pointers: were the size check ever to pass, the entry point's null-pointer
    # check would refuse the call before any launch
    st = a.lib().ivakv_decode_append_attn_noalloc(None, None, None, None, None, None, None,
                                                   None, 8192, 32, 8, 128, 16, 256, 4096,
                                                   0.088, 0, 0, a.F16, None)
    assert st == a.E_WORKSPACE
    assert "static scratch" in a.last_error()
    # 3520 sequences x 8 kv heads (28,160 units) fit, 3600 (28,800) do not
    assert iva.decode_workspace_bytes(3520, 32, 8, 128, 16, 256) <= 64 << 20
    assert iva.decode_workspace_bytes(3600, 32, 8, 128, 16, 256) > 64 << 20
