import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "gpullama3.java_amd"), ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libgpullama3_hip.so)")


def gpu_available():
    """A HIP device is visible to libgpullama3_hip.so (torch is not imported: one HIP runtime per process)."""
    try:
        from gpullama3_hip import device_name
        return bool(device_name())
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip-free guard: a gpu-marked test on a machine without a GPU is an error, not a silent pass."""
    if not gpu_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return True
