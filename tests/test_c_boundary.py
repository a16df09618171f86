"""The boundary from a compiled C caller (tests/c, built by build.py with
tests/c/Makefile): the engine TU (tests/c/engine_tu.c: the engine's own
hook table and the no-backend stubs a maintainer adds) linked without the
library (its stubs decline, the table stays NULL) and with it
(the library fills the engine's own table; the hooks' floors, M gate and
results at BASELINE configs 0 and 1 against the oracle on the GPU box)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "c", "bin")


def run(name, *args):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail("%s not built (__graft_entry__.build() / make -C tests/c)" % path)
    p = subprocess.run([path, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=600)
    print(p.stdout)
    return p


def test_engine_without_backend_links_and_declines():
    p = run("test_nobackend")
    assert p.returncode == 0 and "PASS" in p.stdout


def test_engine_with_backend_on_a_host_without_gpu():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present: test_engine_with_backend_on_gpu covers it")
    p = run("test_boundary")
    assert p.returncode == 0 and "PASS (no device" in p.stdout


@pytest.mark.gpu
def test_engine_with_backend_on_gpu():
    p = run("test_boundary", "--expect-gpu")
    assert p.returncode == 0 and p.stdout.rstrip().endswith("PASS"), p.stdout
