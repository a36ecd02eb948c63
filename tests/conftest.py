import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, TESTS):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PKG_NAME = "comfyui-weightferry_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


def load_pkg():
    """The package, imported by its directory name as ComfyUI imports a custom-node directory."""
    return importlib.import_module(PKG_NAME)


def sub(name):
    return importlib.import_module(f"{PKG_NAME}.{name}")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


def gpu_ready():
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def native():
    """The loaded HIP library (GPU tests): fails loudly when it is not built."""
    n = sub("_native")
    n.lib()
    assert os.path.exists(n.LIB_PATH)
    return n


@pytest.fixture
def fake_gguf():
    """A stand-in ComfyUI-GGUF ops module in sys.modules for the duration of one test."""
    import fake_comfy
    ops = fake_comfy.make_ops_module()
    yield ops
    gd = sub("enhancers.gguf_dequant")
    gd.uninstall()
    fake_comfy.remove_ops_module()
