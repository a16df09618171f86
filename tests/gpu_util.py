"""Device-buffer plumbing for the GPU tests over the HIP runtime that the
backend links (apus-glm5.3-flash_amd/hiprt.py; no torch in GPU processes —
its bundled HIP runtime would be a second runtime in the process)."""
import importlib

import numpy as np


def rt():
    from conftest import load_pkg
    load_pkg()
    return importlib.import_module("apus_ghip.hiprt")


def dev(a):
    """numpy -> device buffer (same bytes)."""
    return rt().DevBuf.of(np.ascontiguousarray(a))


def empty(nbytes):
    return rt().DevBuf(nbytes)


def host(buf, dtype, shape):
    rt().synchronize()
    return buf.download(dtype, shape)


def vp(buf):
    return buf.vp


def stream():
    return None          # the null stream


def download_ptr(ptr, dtype, shape):
    """Copy from a raw device address (e.g. a store slab) to numpy."""
    import ctypes
    r = rt()
    r.synchronize()
    out = np.empty(shape, dtype)
    r.check(r.hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_void_p(ptr), out.nbytes, r.D2H),
            "hipMemcpy D2H")
    return out
