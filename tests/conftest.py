import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


@pytest.fixture(scope="session")
def hip():
    """HipBackend on device 0 (GPU tests only)."""
    from dotllm_amd.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.dispose()


@pytest.fixture(scope="session")
def tiny_image():
    from dotllm_amd import synth
    return synth.build_image("tiny", seed=1234)
