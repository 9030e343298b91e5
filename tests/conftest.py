"""Shared test setup: import paths, the ``gpu`` marker, and the oracle build.

``-m "not gpu"`` tests run anywhere (the CPU oracle, the host logic, the
library's exports); ``-m gpu`` tests need an MI355X and call the HIP library
through its C ABI.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "unlimited-ocr-max_amd"
for p in (ROOT, PKG_DIR):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    if not O.LIB_PATH.exists():
        O.build()
    return O
