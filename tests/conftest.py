import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "flash-hyperconnections_amd"
# FH_TEST_INSTALLED=1: test the flash_hypercons found on sys.path (e.g. a
# `pip install --target DIR .` copy on PYTHONPATH) instead of the source tree.
INSTALLED = os.environ.get("FH_TEST_INSTALLED", "") not in ("", "0")
for path in ((str(ROOT),) if INSTALLED else (str(PKG_DIR), str(ROOT))):
    if path not in sys.path:
        sys.path.insert(0, path)


def _ensure_built():
    """Build the extension and the oracle once if this checkout has none (CPU container)."""
    if not INSTALLED:
        sys.path.insert(0, str(PKG_DIR))
        import build as fh_build  # flash-hyperconnections_amd/build.py

        if not fh_build.built():
            fh_build.build()
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()


_ensure_built()

import torch  # noqa: E402


def _gpu_available() -> bool:
    return torch.cuda.is_available() and torch.version.hip is not None


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct gfx950 GPU (runs the HIP kernels)")
    config.addinivalue_line("markers", "compile: exercises torch.compile")


def pytest_collection_modifyitems(items):
    if not _gpu_available():
        skip = pytest.mark.skip(reason="requires a ROCm gfx950 GPU")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(autouse=True)
def seed():
    torch.manual_seed(9041)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a hard failure still identifies it.
    if "gpu" in request.keywords and os.environ.get("FH_ANNOUNCE", "1") == "1":
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
