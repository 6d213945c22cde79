import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a gfx950 GPU (runs through the C ABI)")


@pytest.fixture(scope="session")
def gpu():
    """The C-ABI library with a gfx950 device; fails (never skips) when the
    device or the built library is missing, so a GPU run cannot pass on a
    silent fallback."""
    import nutllm_amd as nut
    n = nut.device_count()
    assert n > 0, "no gfx950 device visible to libnutllm_hip.so"
    return nut
