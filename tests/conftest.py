from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "cuda: alias kept from the reference suite (GPU required)")


@pytest.fixture(autouse=True)
def _isolated_cache(tmp_path, monkeypatch):
    """Every test gets its own schedule-cache directory."""
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path / "autosage-cache"))
    yield


def gpu_ready() -> bool:
    import torch

    import autosage_amd

    return torch.cuda.is_available() and autosage_amd.load_native() and autosage_amd.native_available()
