"""Test configuration: import paths and the ``gpu`` marker.

``oracle`` (the CPU checker) is imported from the repository root and the
product package ``ragged`` from ragged-mlir_amd/. Tests marked ``gpu`` need a
ROCm device and the built libragged_hip.so; the CPU suite runs with
``-m "not gpu"``.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "ragged-mlir_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def artifact_cache(tmp_path_factory):
    from ragged import ArtifactCache
    return ArtifactCache(tmp_path_factory.mktemp("ragged-cache"))
