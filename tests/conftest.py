import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; run on the GPU box")


@pytest.fixture(scope="session")
def ctx():
    """One device context for the whole GPU session (one process on the card)."""
    from brimkern_amd.capi import Context
    c = Context(0)
    yield c
    c.close()
