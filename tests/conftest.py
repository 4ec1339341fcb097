"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the CPU."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on HIP)")


def load_package():
    """Import lia.rs_amd (the directory name is not a Python identifier)."""
    if "lia_rs_amd" in sys.modules:
        return sys.modules["lia_rs_amd"]
    pkg_dir = os.path.join(ROOT, "lia.rs_amd")
    spec = importlib.util.spec_from_file_location(
        "lia_rs_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lia_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def _ensure_built():
    from oracle import build as ob
    if not os.path.exists(ob.OUT):
        ob.build()
    lib_path = os.path.join(ROOT, "lia.rs_amd", "liblia_hip.so")
    if not os.path.exists(lib_path):
        spec = importlib.util.spec_from_file_location(
            "lia_build", os.path.join(ROOT, "lia.rs_amd", "build.py"))
        m = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(m)
        m.build()


_ensure_built()


@pytest.fixture(scope="session")
def lia():
    return load_package()


@pytest.fixture(scope="session")
def wl():
    load_package()
    import lia_rs_amd.workloads as w
    return w


@pytest.fixture(scope="session")
def O():
    from oracle import oracle
    return oracle
