"""Test configuration: the `gpu` marker, the repo on sys.path, a shared context.

Tests marked ``gpu`` run the HIP library on a gfx950 device and compare it with
the CPU oracle (oracle/). Unmarked tests run on any host without a GPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libsulimo_hip.so")


@pytest.fixture(scope="session")
def ctx():
    from sulimo_amd import hip
    return hip.HipContext.get_or_init(0)
