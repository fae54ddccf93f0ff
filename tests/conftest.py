"""Shared fixtures.  GPU tests carry ``@pytest.mark.gpu``; they FAIL (not skip) when
no GPU is visible, so a broken GPU run cannot pass as skipped."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

IVA = __graft_entry__.load_package()  # registers the package as ``iva_amd``


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


@pytest.fixture(scope="session")
def iva():
    return IVA


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    IVA._abi.lib()  # the HIP library must be built and loadable
    return torch.device("cuda:0")
