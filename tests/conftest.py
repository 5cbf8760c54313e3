"""Shared pytest setup.

* Registers the ``gpu`` marker (tests that need a ROCm device).
* Puts the repository root (for ``oracle``) and the package directory
  ``ojasx-open-source-cuda_amd`` (for ``ojasx_amd``) on ``sys.path``.
* Seeds torch like the reference suite does (``tests/conftest.py:4-6`` of the
  reference seeds 20261006 and uses 2 threads).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "ojasx-open-source-cuda_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


@pytest.fixture(autouse=True)
def _seed():
    import torch

    torch.manual_seed(20261006)
    yield
