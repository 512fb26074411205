"""Shared test setup.

Markers: `gpu` tests need an MI355X (run with -m gpu); everything else runs on
the CPU.  The package directory `dsa-cpu-topk_amd/` holds top-level modules
with the reference's names (dsa_attention, lightning_indexer, ...), so it is
put on sys.path, as a user of the drop-in would.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "dsa-cpu-topk_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP kernels)")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
