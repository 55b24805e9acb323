import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built kernel library")


@pytest.fixture(autouse=True)
def _isolated_popcorn_cache(tmp_path, monkeypatch):
    """Report rows written by a test go to a private cache directory."""
    monkeypatch.setenv("POPCORN_CACHE_DIR", str(tmp_path / "popcorn-cache"))
    monkeypatch.delenv("POPCORN_BENCH", raising=False)
    monkeypatch.delenv("POPCORN_UNSAFE", raising=False)
    yield


def pytest_collection_modifyitems(config, items):
    # GPU tests announce themselves before running so a run that takes the
    # device down still names the case in its output.
    for item in items:
        if item.get_closest_marker("gpu") is not None:
            item.user_properties.append(("gpu", True))


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield
