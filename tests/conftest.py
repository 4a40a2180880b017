import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def hiplib():
    from velox_amd import _lib

    return _lib.load()


class Dev:
    """Device buffers through torch (plumbing only: the kernels under test are the HIP library's)."""

    def __init__(self):
        import torch

        self.torch = torch
        torch.cuda.init()

    def put(self, a: np.ndarray):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to("cuda")

    def empty(self, n: int, dtype=np.float32):
        tdt = {np.float32: self.torch.float32, np.uint32: self.torch.int32, np.uint8: self.torch.uint8,
               np.uint16: self.torch.int16}[dtype]
        return self.torch.zeros(n, dtype=tdt, device="cuda")

    def get(self, t, dtype=None) -> np.ndarray:
        self.torch.cuda.synchronize()
        a = t.cpu().numpy()
        return a.view(dtype) if dtype is not None else a


@pytest.fixture(scope="session")
def dev():
    return Dev()
