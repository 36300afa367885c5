"""Shared test setup: import paths, the `gpu` marker and a GPU context."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "hale-token_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (run on the MI355X box)")


@pytest.fixture(scope="session")
def ctx():
    """One GPU context for the whole session (tests marked gpu only)."""
    import hale_moe

    c = hale_moe.Context(0)
    yield c
    c.close()
