import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs on the GPU box (pytest -m gpu)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP runtime with one visible device. GPU tests skip only when no
    device exists; a missing native library is an error, not a skip."""
    from windlass_amd import hip, moe
    moe.load()  # raises NativeLibraryMissing: there is no fallback path
    if hip.device_count() < 1:
        pytest.skip("no GPU visible")
    return hip
