"""Test configuration: the repo root on sys.path and the `gpu` marker.

Tests marked `gpu` need an MI355X and the built library (they fail, not skip, without one);
the rest run on any CPU.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")

