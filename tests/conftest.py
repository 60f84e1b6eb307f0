import importlib
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (str(REPO), str(REPO / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libw4a8_mi355x.so")


def pkg(sub: str = ""):
    name = "minisglang-rdna4_amd" + (("." + sub) if sub else "")
    return importlib.import_module(name)


@pytest.fixture(scope="session")
def kernels():
    return pkg("quant.kernels")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.build()
    return o


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected but no HIP device is visible")
    return torch.device("cuda:0")
