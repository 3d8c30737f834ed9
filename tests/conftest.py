import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def _gpu_present():
    # The kernel driver's node; checking it initialises nothing on the GPU.
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def gpu():
    if not _gpu_present():
        pytest.skip("no GPU on this host")
    from chattorrent_amd import ccdecode
    return ccdecode.load()
