"""Test configuration: import paths, the ``gpu`` marker and shared helpers."""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "iris-3b-metal_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available() and os.environ.get("IRIS_SKIP_GPU_TESTS") != "1":
        return
    skip = pytest.mark.skip(reason="needs a GPU (or IRIS_SKIP_GPU_TESTS=1)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
