"""pytest configuration: the `gpu` marker and shared fixtures.

`-m "not gpu"` runs the oracle, host-logic and ABI tests on the CPU; `-m gpu` runs the parity tests through the C-ABI
library on an MI355X.  GPU tests are skipped (not failed) on a machine without a GPU; on a GPU machine a missing
native library fails them (neural_amd has no fallback).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU on this machine")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
