"""Shared test set-up: import paths, the ``gpu`` marker, seeded helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "triton-transformer-kernels_amd"
for path in (str(REPO), str(PKG)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library"
    )


def pytest_collection_modifyitems(config, items):
    # GPU tests must fail loudly (not skip) on a GPU box whose library is
    # missing; on a machine without a GPU they are deselected with -m "not gpu".
    pass


@pytest.fixture(scope="session")
def gpu_ready():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible ROCm device")
    from transformer_opt import _native

    _native.load()  # raises when the HIP library is missing
    return True
