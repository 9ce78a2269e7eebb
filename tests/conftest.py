"""Shared pytest setup: the `gpu` marker, in-tree build on demand, and the
device/stream fixtures of the GPU parity tests."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    from yuuka_amd import build as b
    b.ensure_built()


_ensure_built()


@pytest.fixture(scope="session")
def dev():
    from yuuka_amd import hip
    d = hip.Device(0)
    yield d
    d.close()


@pytest.fixture(scope="session")
def stream(dev):
    from yuuka_amd import hip
    s = hip.Stream(dev)
    yield s
    s.destroy()
