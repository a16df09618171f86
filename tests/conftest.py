"""Shared test fixtures.

CPU tests (-m "not gpu") pin the oracle (oracle/) against the reference's
known-answer tests, closed forms, independent numpy restatements, the
committed golden fixtures and, where it was built, the reference's own CPU
kernels (oracle/_ref). GPU tests (-m gpu) compare the HIP backend, called
through its C ABI, with the oracle on the same inputs.
"""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def load_pkg():
    path = os.path.join(ROOT, "apus-glm5.3-flash_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(
        "apus_ghip", path,
        submodule_search_locations=[os.path.dirname(path)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules.setdefault("apus_ghip", mod)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def ghip(pkg):
    """The backend library, enabled on the GPU (GPU tests only)."""
    import ctypes
    lib = pkg.load()
    buf = ctypes.create_string_buffer(256)
    rc = lib.apus_ghip_enable(buf, 256)
    if rc != 0:
        pytest.fail("apus_ghip_enable failed: %s" % buf.value.decode())
    return lib
