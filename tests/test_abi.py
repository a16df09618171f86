"""The C-ABI library builds, loads and exports every symbol that
include/*.h declares; the ctypes signature table covers the same set; on a
host without a GPU the backend declines cleanly (no compute is issued)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for fn in os.listdir(INCLUDE):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"\(\*\w+\)\([^)]*\)", "", text)   # hook member types
        for m in re.finditer(r"\b(apus_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path],
                         stdout=subprocess.PIPE, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def test_every_declared_symbol_is_exported(pkg):
    decl = declared_functions()
    assert len(decl) >= 40
    ex = exported(pkg.LIB_PATH)
    missing = sorted(decl - ex)
    assert not missing, missing
    assert "apus_ghip_hooks" in ex                # the hook table object


def test_signature_table_matches_headers(pkg):
    assert declared_functions() == set(pkg.SIGNATURES)


def test_loads_and_declines_without_gpu(pkg):
    lib = pkg.load()
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present: the GPU suite covers enable")
    buf = ctypes.create_string_buffer(256)
    assert lib.apus_ghip_enable(buf, 256) != 0
    assert buf.value                               # a reason is given
    assert lib.apus_ghip_is_enabled() == 0
    hooks = (ctypes.c_void_p * 2).in_dll(lib, "apus_ghip_hooks")
    assert hooks[0] is None and hooks[1] is None  # fail-soft: CPU kernels run
    assert lib.apus_ghip_register_region(None, 0) != 0
