"""Test configuration: the ``gpu`` marker, the repository root on ``sys.path``."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) device and the built HIP library")


@pytest.fixture(autouse=True)
def _fresh_log_state():
    from foldforge_amd import dispatch

    dispatch.forget_announcements()
    yield
