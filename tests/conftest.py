"""Test configuration: markers, package loading, GPU helpers.

The product directory ``comfyui-applesilicon-optimized_amd`` is a ComfyUI
custom-node package (a directory name that is not a Python identifier); it is
loaded here under the module name ``cdna4q`` the way ComfyUI loads custom
nodes, by path.
"""
import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "comfyui-applesilicon-optimized_amd"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    if "cdna4q" in sys.modules:
        return sys.modules["cdna4q"]
    spec = importlib.util.spec_from_file_location(
        "cdna4q", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["cdna4q"] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built libcdna4q.so")
    config.addinivalue_line("markers", "slow: long CPU-only check")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)
