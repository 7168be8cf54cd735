"""Shared pytest setup: the `gpu` marker, loaders for the package and the oracle."""
from __future__ import annotations

import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def load_package():
    """Import trellis.cpp_amd/ as the module `trellis_cpp_amd` (the directory name holds a
    dot, so it is loaded by path)."""
    if "trellis_cpp_amd" in sys.modules:
        return sys.modules["trellis_cpp_amd"]
    pkg_dir = os.path.join(ROOT, "trellis.cpp_amd")
    spec = importlib.util.spec_from_file_location(
        "trellis_cpp_amd", os.path.join(pkg_dir, "__init__.py"),
        submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["trellis_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


# the package is importable as trellis_cpp_amd from every test module (the library itself loads
# lazily, on the first device call)
load_package()


def load_oracle():
    if "trellis_oracle" in sys.modules:
        return sys.modules["trellis_oracle"]
    spec = importlib.util.spec_from_file_location(
        "trellis_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["trellis_oracle"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def shells(pkg):
    import trellis_cpp_amd.shells as s
    return s


@pytest.fixture(scope="session")
def orc():
    return load_oracle()


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def _load(name):
        with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
            return {k: z[k] for k in z.files}
    return _load


@pytest.fixture(scope="session")
def gpu_lib(pkg):
    """The HIP library on a GPU; skips GPU tests when no GPU is visible, and fails loudly when
    a GPU is present but the library is not built."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    pkg.lib()   # raises if libtrellis_sparse.so is missing
    return pkg
