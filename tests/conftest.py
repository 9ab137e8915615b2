"""Shared fixtures and markers.

``gpu``-marked tests need an MI355X (gfx950) and the built kernel library; they are skipped
when no GPU is visible. Everything else runs on CPU: the oracle, the host-side policy code
(dispatch, config, autotune cache, metrics) and the C-ABI library's exported symbols.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

_HAS_GPU = torch.cuda.is_available()


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running; excluded from the quick tiers")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    skip_gpu = pytest.mark.skip(reason="needs a gfx950 GPU")
    for item in items:
        if "gpu" in item.keywords and not _HAS_GPU:
            item.add_marker(skip_gpu)


@pytest.fixture(scope="session")
def device() -> torch.device:
    if not _HAS_GPU:
        pytest.skip("needs a gfx950 GPU")
    return torch.device("cuda")


@pytest.fixture(autouse=True)
def _isolated_cache_dir(tmp_path_factory: pytest.TempPathFactory, monkeypatch: pytest.MonkeyPatch):
    """Every test gets its own autotune cache dir; nothing leaks into ~/.cache."""
    monkeypatch.setenv("TOKENFORGE_CACHE_DIR", str(tmp_path_factory.mktemp("tf-cache")))
    from tokenforge.kernels import autotune

    autotune.reset_caches()
    yield
    autotune.reset_caches()
