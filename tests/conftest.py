"""Test configuration: import paths, the `gpu` marker and the test-only vLLM stand-in."""
import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "vllm-quant-kernels_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

# vLLM is not installed in this image: use the minimal stand-in under tests/fake_vllm.
if importlib.util.find_spec("vllm") is None:
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "fake_vllm"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) GPU and libvqk_hip.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
