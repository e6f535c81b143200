import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


def pytest_collection_modifyitems(config, items):
    # torch's HIP runtime first: libfish_hip.so (loaded by ctypes) and torch must share one
    # runtime, and it is the first one loaded that the process keeps, whatever order the
    # selected tests run in
    if any(item.get_closest_marker("gpu") for item in items):
        import torch
        torch.cuda.is_available()


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    d = os.path.join(ROOT, "tests", "golden")

    def load(name):
        return np.load(os.path.join(d, name + ".npz"), allow_pickle=False)

    return load
