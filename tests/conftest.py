import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libqwhip.so")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (a GPU test fails loudly when
    the library or the device is missing: there is no CPU fallback)."""
    import qwenscriber_amd as qa

    context = qa.Context(0)
    yield context
    context.close()
