import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "universal-ai-inference_amd"))
sys.path.insert(0, str(ROOT))

os.environ.setdefault("UAII_MODEL_CACHE", "/tmp/uaii_models")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def hip():
    """libuaii_amd.so with the HIP device initialised (GPU tests only)."""
    import uaii_amd
    L = uaii_amd.lib()
    n = __import__("ctypes").c_int(0)
    rc = L.uaii_hip_device_count(__import__("ctypes").byref(n))
    if rc != 0 or n.value < 1:
        raise RuntimeError("no HIP device visible to libuaii_amd.so")
    uaii_amd.check_hip(L.uaii_hip_init(0), "init")
    return L
