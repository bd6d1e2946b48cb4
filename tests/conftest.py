"""Shared test setup: import paths, the `gpu` marker, a session GPU context."""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "gemma-4-webgpu-kernels_amd"
for p in (str(PKG), str(REPO / "oracle"), str(REPO / "tests" / "golden"), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels through the C-ABI")


@pytest.fixture(scope="session")
def ctx():
    """One g4a context for the whole GPU session (fails loudly if the library or device is missing)."""
    import g4a
    c = g4a.Context(0)
    info = c.device_info()
    print(f"\n[g4a] device {info.device}: {info.arch.decode()} with {info.compute_units} CUs", flush=True)
    yield c
    c.close()
