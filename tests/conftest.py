import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "ir-multivector-retrieval_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950)")


def gpu_available() -> bool:
    try:
        from tac_gpu import device
    except ImportError:
        return False
    return device.device_count() > 0


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from tac_gpu import errors, lib
    errors.check(lib.tac_gpu_set_device(0))
    return True
