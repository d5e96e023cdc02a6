import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "forge-llm_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the device)")


@pytest.fixture(scope="session")
def fh():
    """The C ABI, initialised on device 0 (GPU tests only)."""
    import forge_hip
    if forge_hip.device_count() < 1:
        pytest.skip("no GPU visible")
    forge_hip.init(0)
    return forge_hip
