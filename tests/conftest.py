"""Shared test setup: the `gpu` marker, loaders for the product library and the CPU oracle."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
if ORACLE_DIR not in sys.path:
    sys.path.insert(0, ORACLE_DIR)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def load_product():
    """Imports the package in ds-ocr_amd/ (the directory name is not an identifier)."""
    name = "ds_ocr_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "ds-ocr_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _ensure_oracle_built():
    lib = os.path.join(ORACLE_DIR, "liboracle.so")
    if not os.path.exists(lib):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


_ensure_oracle_built()


@pytest.fixture(scope="session")
def B():
    import bindings
    return bindings


@pytest.fixture(scope="session")
def lib():
    return load_product()


@pytest.fixture(scope="session")
def dev(lib):
    """The loaded product library with the device initialised (GPU tests)."""
    L = lib.load()
    rc = L.ds_hip_init()
    if rc != 0:
        raise RuntimeError("HIP init failed: " + L.ds_hip_last_error().decode())
    return lib
