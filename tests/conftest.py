import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "frame-public_amd")
for p in (PKG, os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs the HIP path through the C ABI")


@pytest.fixture(scope="session")
def hip():
    """The kernel library's ctypes binding. On a GPU box a missing library or device is a failure, not a skip."""
    from frame_hip import abi

    lib = abi.lib()
    n = abi.device_count()
    assert n >= 1, "no HIP device visible"
    print(f"[gpu] devices={n} abi_version={lib.fh_abi_version()}", flush=True)
    return abi
