"""Shared fixtures. GPU tests are marked `gpu` and need a gfx950 device plus the built library;
they fail loudly (never skip) when the library is missing, so a GPU run cannot pass on a
fallback."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


@pytest.fixture
def runtime():
    from tessery_amd import HipRuntime

    with HipRuntime() as engine:
        yield engine


GOLDEN = ROOT / "tests" / "golden"
