import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libh3hip.so")


@pytest.fixture(scope="session")
def gpu():
    """One device context for the whole GPU session. The product path has no CPU fallback: if the
    library or the device is missing this fixture raises, and every GPU test fails loudly."""
    from h3metal_amd.gpu import Gpu
    g = Gpu()
    print(f"\n[gpu] {g.device}", flush=True)
    yield g
    g.close()
