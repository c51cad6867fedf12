"""pytest set-up: the `gpu` marker, import paths for the ctypes binding and the oracle, a session-wide device."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "p0pc0rn-kernels_amd", "python"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs on the GPU box")


@pytest.fixture(scope="session")
def dev():
    import p0k
    d = p0k.Device(0)
    print(f"[p0k] device {d.info()}", flush=True)
    yield d
    d.close()
