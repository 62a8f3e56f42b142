"""Shared fixtures: the native library harness and the CPU oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_mx():
    """Import rust-mlx_amd (hyphenated directory) as module `rust_mlx_amd`."""
    if "rust_mlx_amd" in sys.modules:
        return sys.modules["rust_mlx_amd"]
    path = os.path.join(ROOT, "rust-mlx_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location("rust_mlx_amd", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rust_mlx_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def mx():
    return load_mx()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    return oracle
