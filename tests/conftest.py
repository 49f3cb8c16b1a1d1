"""pytest setup: import paths, the `gpu` marker, and skipping GPU tests on GPU-less hosts."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "rotorquant-vllm_amd"), os.path.join(ROOT, "oracle"), os.path.dirname(__file__),
          os.path.join(os.path.dirname(__file__), "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built librq_hip.so")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
