import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "inkling-fa4-relative-attention_amd")
for p in (REPO, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    lib = os.path.join(PKG_DIR, "inkling_fa4", "libifa4.so")
    ext = os.path.join(PKG_DIR, "inkling_fa4", "_ifa4_torch.so")
    if not (os.path.exists(lib) and os.path.exists(ext)):
        import importlib.util

        spec = importlib.util.spec_from_file_location("_ifa4_build", os.path.join(PKG_DIR, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()


_ensure_built()


@pytest.fixture(scope="session")
def cuda():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")
