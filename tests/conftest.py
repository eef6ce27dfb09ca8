"""Shared pytest setup: the `gpu` marker, import paths, and a session-wide
device context for the GPU tests."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("mimir-framework_amd", "oracle", "tests"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmimir_hip on cuda:0)")


@pytest.fixture(scope="session")
def ctx():
    import mimir_hip
    c = mimir_hip.Context(0)
    yield c
    c.close()
