"""Every shipped gfx950 kernel instantiation runs without scratch (register spills to
per-lane memory): the compiler's kernel-resource-usage remarks report ScratchSize 0 for
each kernel of every source under iva1.0_amd/csrc (a device-only compile, no GPU)."""
from __future__ import annotations

import pytest


@pytest.fixture(scope="module")
def usage(iva):
    from importlib import import_module
    return import_module("iva_amd.build").kernel_resource_usage()


def test_every_kernel_was_reported(usage):
    names = " ".join(usage)
    for kernel in ("decode_stream_kernel", "decode_partial_kernel", "decode_fused_merge_kernel",
                   "prefill_kernel", "append_kernel", "gather_kernel", "copy_pages_kernel",
                   "append8_kernel", "rope_kernel"):
        assert kernel in names, f"no resource remark for {kernel}"
    assert all("ScratchSize" in v and "VGPRs" in v for v in usage.values())
    assert len(usage) >= 100


def test_no_kernel_uses_scratch(usage):
    spilling = {k: v["ScratchSize"] for k, v in usage.items() if v["ScratchSize"] != 0}
    assert not spilling, f"kernels with scratch (bytes/lane): {spilling}"
