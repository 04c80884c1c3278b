import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950) and the built backend")


@pytest.fixture(scope="session")
def ctx():
    """One backend context on device 0 for the whole session; the backend
    library must be built (there is no other implementation to fall back to)."""
    from beatlm_amd import hip

    try:
        c = hip.Context(0)
    except hip.BackendError as e:
        pytest.skip(f"no GPU visible: {e}")
    yield c
    c.close()
