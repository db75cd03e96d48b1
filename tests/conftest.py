"""Test configuration: import paths and the `gpu` marker.

`-m gpu` tests need an MI355X and call the HIP library through its C ABI;
everything else runs on the CPU (oracle pinning, host logic, ABI exports).
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "s4000-moe-engine_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and libkvc.so")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def deterministic_decode(monkeypatch):
    """Paged decode without the dynamic tail hand-out (KVC_DECODE_STEAL=0):
    which workgroup takes which tail tile depends on timing, and with it the
    fp32 summation order of a split row, so bitwise comparisons of two
    launches' outputs need the static partition alone.  Pool bytes are
    bit-exact either way."""
    monkeypatch.setenv("KVC_DECODE_STEAL", "0")
