"""Test configuration: the ``gpu`` marker and the repo root on ``sys.path``.

``-m "not gpu"`` runs the CPU suite (oracle pinning, host logic, C-ABI exports); ``-m gpu``
runs the parity tests that call the HIP kernels through the C ABI. GPU tests are skipped only
when no HIP device is visible -- a missing kernel library is a failure, not a skip.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device; calls the kernels through the C ABI")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
