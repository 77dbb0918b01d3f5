import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_NAME = "comfyui-int4-convrot-rdna4_amd"
for p in (ROOT, os.path.join(ROOT, "tests", "golden"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def import_pkg():
    return importlib.import_module(PKG_NAME)


def import_backend():
    import_pkg()
    return importlib.import_module(PKG_NAME + "._int4")


@pytest.fixture(scope="session")
def backend():
    return import_backend()


@pytest.fixture(scope="session")
def native(backend):
    return importlib.import_module(PKG_NAME + "._int4.native")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    return O


@pytest.fixture(scope="session")
def goldens():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "goldens.npz"))


@pytest.fixture(scope="session")
def gpu(native):
    """Skip-free GPU gate: a gpu-marked test on a machine without the GPU or
    the library fails loudly instead of silently passing."""
    import torch
    assert torch.cuda.is_available(), "gpu tests need a visible MI355X"
    assert native.is_available(), "libconvrot_gfx950.so not loadable or device is not gfx950"
    return torch.device("cuda")
