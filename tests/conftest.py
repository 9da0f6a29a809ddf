"""Test configuration: the `gpu` marker, import paths, and index validation in Ops.

GPU tests run on an MI355X (`pytest -m gpu`); everything else runs on the CPU
(`pytest -m "not gpu"`). GPU tests are skipped where no GPU is visible."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

# Ops checks every block id / tail slot against the buffers before a launch (one host sync):
# a wrong index in a test then raises instead of reaching a kernel.
os.environ.setdefault("KUSHKASH_AMD_VALIDATE", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
