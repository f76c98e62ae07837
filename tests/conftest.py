import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def device():
    from furykernel_amd import runtime

    dev = runtime.Device(0)
    yield dev
    dev.close()


@pytest.fixture(scope="session")
def kernels(device):
    from furykernel_amd.kernels import Kernels

    return Kernels(device)


@pytest.fixture(scope="session")
def golden():
    import json

    return lambda name: json.loads((ROOT / "tests" / "golden" / name).read_text())
