"""Test configuration: registers the ``gpu`` marker and the repo root on
sys.path.  GPU tests require the in-tree ``mote_amd/libmote_hip.so`` and a
visible device; they fail (never skip) when either is missing, so a silent
fallback can never pass them."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run on the GPU box")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def stream():
    from mote_amd import device

    if device.device_count() < 1:
        pytest.fail("no HIP device visible to a test marked gpu")
    s = device.Stream()
    yield s
    s.close()
