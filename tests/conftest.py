"""Test configuration: the `gpu` marker, repo on sys.path, the native library built once.

CPU tests (-m "not gpu") cover the oracle, the host logic and the C ABI's exports;
GPU tests (-m gpu) run the HIP path on a gfx950 device and check it against the
oracle.
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs the HIP kernels)")


@pytest.fixture(scope="session", autouse=True)
def native_library():
    """Build libffn_mi355x.so and the C oracle if they are absent (never rebuilt here)."""
    from ffn_optim_amd import _lib
    if not _lib.LIBRARY_PATH.exists():
        from ffn_optim_amd.build import build
        build()
    from oracle import build as oracle_build
    if not oracle_build.LIBRARY.exists():
        oracle_build.build()
    return _lib.load()
