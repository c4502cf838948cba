"""pytest configuration: the `gpu` marker, and building what the tests load.

Tests load the in-tree builds (darknet_zig_amd/libdkz.so, oracle/libdkz_oracle.so,
tests/native/libdkz_checks.so) and build only what is missing.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


def _ensure_built() -> None:
    from darknet_zig_amd import _lib
    from darknet_zig_amd import build as pkg_build
    from oracle import ref
    from tests.native import build as native_build

    if not _lib.LIB_PATH.exists():
        pkg_build.build()
    if not ref.LIB_PATH.exists():
        ref.build()
    if not native_build.LIB.exists():
        native_build.build()
    if not native_build.GPUTEST.exists():
        native_build.build_gputest()


_ensure_built()


@pytest.fixture(scope="session")
def dev():
    """Initialises device 0 with sync-after-launch on, as gputest does
    (gputest.zig:64-69), so a faulting kernel is named by its own op."""
    from darknet_zig_amd import gpu

    gpu.init(0)
    gpu.setSyncAfterLaunch(True)
    yield gpu
    gpu.sync()
