"""Test setup: import paths for the package and the oracle, and the ``gpu`` marker.

``-m "not gpu"`` runs on a CPU-only host (oracle pinning, host planner, C-ABI exports);
``-m gpu`` tests need a ROCm GPU and call the HIP kernels through ``libvdnh3.so``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "comfyui-kirei-vdn-h3_amd"
for p in (str(ROOT), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libvdnh3.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def built_lib():
    """The loaded libvdnh3.so; it is built here only if no built copy exists."""
    from vdn_h3_amd import _build, _lib

    if not _lib.LIB_PATH.exists():
        _build.build()
    return _lib.lib()
