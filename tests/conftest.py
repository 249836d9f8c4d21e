import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "deepseek-on-one-gpu_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libamla.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    from safetensors.torch import load_file
    import json
    d = os.path.join(ROOT, "tests", "golden")
    tensors = load_file(os.path.join(d, "reference_vectors.safetensors"))
    with open(os.path.join(d, "reference_vectors.json")) as f:
        manifest = json.load(f)
    return tensors, manifest
