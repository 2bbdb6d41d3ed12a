"""Shared pytest configuration: the `gpu` marker and repository import paths."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any(item.get_closest_marker("gpu") for item in items) and not _gpu_available():
        skip = pytest.mark.skip(reason="no GPU visible")
        for item in items:
            if item.get_closest_marker("gpu"):
                item.add_marker(skip)
