import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "project-obsidian_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def exe():
    """One HIP context for all GPU tests (no fallback: fails if the library
    or the device is missing)."""
    import obsidian_hip as oh

    e = oh.ObsidianExecutor(0)
    yield e
    e.close()


@pytest.fixture(scope="session")
def orc():
    import oracle

    return oracle
