"""Shared test set-up: the `gpu` marker, package / oracle loaders."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "kvmem-llama.cpp_amd"
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def load_pkg():
    """Import kvmem-llama.cpp_amd/ as module `kvmem_amd` (building the
    library first only if nothing is built)."""
    if "kvmem_amd" in sys.modules:
        return sys.modules["kvmem_amd"]
    if not (PKG_DIR / "libkvmem_hip.so").exists():
        import subprocess
        subprocess.run([sys.executable, str(PKG_DIR / "build.py")], check=True)
    spec = importlib.util.spec_from_file_location(
        "kvmem_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["kvmem_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def kv():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle():
    import kvmem_oracle
    kvmem_oracle.lib()
    return kvmem_oracle


@pytest.fixture(scope="session")
def ctx(kv):
    c = kv.Context(0)
    yield c
    c.sync()
    c.close()
