"""Shared pytest setup: the `gpu` marker, the repo on sys.path, and the
session-wide device context for GPU tests."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def load_golden(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


@pytest.fixture(scope="session")
def ctx():
    """Device 0 context. Fails (does not skip) when the library or the GPU is
    missing: a GPU test must never pass without running the HIP path."""
    from inferc_amd.rt import Context

    c = Context(0)
    yield c
    c.close()
