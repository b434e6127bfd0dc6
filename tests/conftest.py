import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

import __graft_entry__ as entry  # noqa: E402
from oracle import oracle as orc  # noqa: E402  (the checker)

pkg = entry.load_package()
capi = pkg.capi
wl = pkg.workloads


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")


def pytest_collection_modifyitems(config, items):
    gpu_ok = None
    for item in items:
        if "gpu" in item.keywords:
            if gpu_ok is None:
                import torch
                gpu_ok = torch.cuda.is_available()
            if not gpu_ok:
                item.add_marker(pytest.mark.skip(reason="no HIP GPU in this environment"))


@pytest.fixture(scope="session")
def oracle():
    orc.lib()
    return orc


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available()
    capi.lib()  # loud failure if the HIP library is missing
    return torch.device("cuda:0")
