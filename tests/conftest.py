import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
TESTS = pathlib.Path(__file__).resolve().parent
if str(TESTS) not in sys.path:
    sys.path.insert(0, str(TESTS))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib


@pytest.fixture(scope="session")
def vx():
    """The product library; GPU tests fail loudly when it is not built."""
    from voxcpm_amd import ops
    from voxcpm_amd._lib import lib
    lib()
    return ops


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    name = torch.cuda.get_device_properties(0).gcnArchName
    print(f"device: {name}", flush=True)
    return torch.device("cuda:0")


@pytest.fixture
def stream(cuda):
    import torch
    s = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(s):
        yield s
    s.synchronize()


def threads() -> int:
    return min(16, os.cpu_count() or 1)
