import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libweft_hip")


@pytest.fixture(scope="session")
def hip():
    """The GPU harness: torch on cuda:0 plus libweft_hip through its C ABI."""
    from tests import _hip
    return _hip.Harness()
