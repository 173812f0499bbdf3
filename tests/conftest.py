"""Test configuration.

Two kinds of tests:
- `gpu`-marked: parity tests on a real MI355X; they call the gfx950 library
  through its C ABI (or the mojo device) and compare with the oracle.
- unmarked: CPU-only.  They check the oracle, the library's exports and the
  host-side device layer.  Without a GPU the device layer runs on the host
  stand-in of the library (tests/host_standin.py); with a GPU it runs on the
  real library.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "torch-mojo-backend_amd"
for p in (str(ROOT), str(PKG), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("TORCH_MOJO_BACKEND_TESTING", "1")

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (gfx950)")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


_MODE = None


def setup_mojo() -> str:
    """Register the mojo device once per process; returns "gpu" or "host"."""
    global _MODE
    if _MODE is not None:
        return _MODE
    from torch_mojo_backend.mojo_device import torch_mojo_tensor as tm
    from torch_mojo_backend import eager_kernels as ek

    if HAS_GPU:
        ek.lib()  # must load: no fallback
        _MODE = "gpu"
    else:
        import host_standin

        tm.set_storage_kind_for_tests("cpu")
        ek.set_library_for_tests(host_standin.HostStandIn())
        _MODE = "host"
    from torch_mojo_backend import register_mojo_devices

    register_mojo_devices()
    return _MODE


@pytest.fixture(scope="session")
def mojo():
    return setup_mojo()


@pytest.fixture(scope="session")
def kernels():
    """The real gfx950 library (GPU tests only)."""
    if not HAS_GPU:
        pytest.skip("no GPU")
    from torch_mojo_backend import eager_kernels as ek

    return ek.lib()
