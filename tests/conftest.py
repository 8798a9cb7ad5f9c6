"""Shared test setup: the `gpu` marker, import paths, and the two libraries under test."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma4-webgpu-engine_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o  # the CPU restatement (test infrastructure)
    o.lib()
    return o


@pytest.fixture(scope="session")
def g4():
    import g4w8a8
    g4w8a8.lib()
    return g4w8a8


@pytest.fixture(scope="session")
def gpu(g4):
    """The HIP library on a live device. Fails (does not skip) when there is none: a GPU test that
    cannot reach the device has not passed."""
    n = g4.device_count()
    assert n > 0, "no HIP device visible to the GPU tests"
    g4.lib().g4_set_device(0)
    return g4
