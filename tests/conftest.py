"""Test setup: import paths, the ``gpu`` marker, shared helpers.

``-m "not gpu"`` runs on any machine: the oracle against its pins, the
registry/platform logic, and the C-ABI library's exports (no device calls).
``-m gpu`` runs on an MI355X: every HIP kernel against the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "dexter-labs_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def built_lib():
    """Path of the built shared library; builds it first if it is missing."""
    from dexter_amd.ops.gfx950 import _lib
    if not _lib.LIB_PATH.exists():
        sys.path.insert(0, str(ROOT / "dexter-labs_amd" / "csrc"))
        import build  # noqa: WPS433 (csrc/build.py)
        build.build()
    return _lib.LIB_PATH
