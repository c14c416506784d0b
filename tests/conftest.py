"""Shared fixtures. `gpu` marks tests that need an MI355X (gfx950) device."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the MI355X box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    return pyoracle.lib()


@pytest.fixture(scope="session")
def P():
    from oracle import pyoracle

    return pyoracle.p


@pytest.fixture(scope="session")
def ctx():
    """The GPU context (gpu tests only). Fails loudly if the device is absent."""
    from franken_ocr_amd.device import default_context

    c = default_context(0)
    info = c.info()
    print(f"[gpu] device {info}", flush=True)
    return c


@pytest.fixture
def rng():
    return np.random.default_rng(0xF0C0)
