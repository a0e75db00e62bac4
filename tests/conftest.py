"""Test configuration: import paths, the `gpu` marker, and the library/GPU fixtures.

`pytest -m "not gpu"` runs the oracle pins, host logic and C-ABI checks on the CPU. `pytest -m gpu` runs the parity
tests on a HIP device; there they fail (not skip) when the library is missing, so a silent fallback cannot pass.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "attention-lab_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libattnlab.so")


def _has_gpu() -> bool:
    import torch
    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def native_lib():
    """The loaded libattnlab.so; built in-tree first when it is missing (the CPU container has no prebuilt copy)."""
    from attention_lab import _native
    if not os.path.exists(_native.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build_library()
    return _native.lib()


@pytest.fixture(scope="session")
def gpu(native_lib):
    """cuda:0 with the HIP library loaded; fails loudly when either is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU test without a HIP device"
    from attention_lab import _native
    assert _native.gpu_available(), "libattnlab.so did not load on the GPU box"
    return torch.device("cuda:0")
