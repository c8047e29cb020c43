"""Shared pytest configuration.

Tests marked ``gpu`` need a HIP device; everything else runs on the CPU.
The product libraries and the oracle are built in-tree by
``__graft_entry__.build()``; a session that finds nothing built builds once.
"""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.join(ROOT, "tests")
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers",
                            "gpu: needs a HIP device (MI355X / gfx950)")


def _load_package():
    spec = importlib.util.spec_from_file_location(
        "m3c_amd", os.path.join(ROOT, "m3.c_amd", "__init__.py"))
    module = importlib.util.module_from_spec(spec)
    sys.modules["m3c_amd"] = module
    spec.loader.exec_module(module)
    return module


def _ensure_built():
    product = [os.path.join(ROOT, "m3.c_amd", name)
               for name in ("libm3.so", "libm3_hip.so")]
    oracle = os.path.join(ROOT, "oracle", "liboracle.so")
    if not all(os.path.exists(p) for p in product):
        subprocess.run(["make", "-C", os.path.join(ROOT, "m3.c_amd"),
                        "-j8"], check=True, stdout=subprocess.DEVNULL)
    if not os.path.exists(oracle):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "all"],
                       check=True, stdout=subprocess.DEVNULL)


_ensure_built()
m3 = _load_package()


@pytest.fixture(scope="session")
def m3pkg():
    return m3


@pytest.fixture(scope="session")
def hip_available():
    return m3.hip_device_count() > 0


@pytest.fixture(scope="session")
def gpu(hip_available):
    if not hip_available:
        pytest.fail("test is marked gpu but no HIP device is visible; the "
                    "HIP provider must run here")
    return True
