import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle_lib  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def load_qk_module():
    """The binding module lives in a directory whose name is not a Python identifier."""
    path = os.path.join(ROOT, "qwen3.8_27b_reference_amd", "qk.py")
    spec = importlib.util.spec_from_file_location("qk_binding", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def qkmod():
    return load_qk_module()


@pytest.fixture(scope="session")
def qk(qkmod):
    return qkmod.Lib()


@pytest.fixture(scope="session")
def oracle():
    o = oracle_lib.Oracle()
    o.init(min(8, os.cpu_count() or 1))
    return o


@pytest.fixture(scope="session")
def reflib():
    if not oracle_lib.ref_available():
        pytest.skip("oracle/_ref not built or host lacks AVX-512")
    r = oracle_lib.RefLib()
    r.init(min(8, os.cpu_count() or 1))
    return r


def load_hiprt_module():
    path = os.path.join(ROOT, "qwen3.8_27b_reference_amd", "hiprt.py")
    spec = importlib.util.spec_from_file_location("qk_hiprt", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def hiprt():
    return load_hiprt_module()


@pytest.fixture(scope="session")
def hip(hiprt):
    h = hiprt.Hip()
    if h.device_count() < 1:
        raise RuntimeError("GPU test run without a visible GPU")
    return h


class Dev:
    """Device buffers for the tests (plumbing only): put/empty return hiprt.Buf objects."""

    def __init__(self, hip, hiprt):
        self.hip = hip
        self.Buf = hiprt.Buf

    def put(self, a):
        return self.Buf.of(self.hip, a)

    def empty(self, nbytes):
        return self.Buf(self.hip, nbytes)

    def stream(self):
        return 0


@pytest.fixture(scope="session")
def dev(hip, hiprt):
    return Dev(hip, hiprt)
