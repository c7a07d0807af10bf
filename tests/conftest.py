"""pytest configuration: import paths and the ``gpu`` marker.

``graph-kernel-injection_amd/`` is the source root of the product (it holds
the ``gki`` package and the drop-in modules ``sparse_triton_kernel`` /
``fx_compiler_pass``); the repo root gives access to ``oracle``.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "graph-kernel-injection_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
