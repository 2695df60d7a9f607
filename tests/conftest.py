"""Shared test setup: repo root on sys.path, the ``gpu`` marker, and helpers.

``-m "not gpu"`` runs the CPU suite (oracle pins, SDK, pack loader, IR
passes, compiler planning for gfx950 without a device, C-ABI exports);
``-m gpu`` runs the parity tests on an MI355X through the C ABI.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP kernels")
