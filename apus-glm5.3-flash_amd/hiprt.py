"""Minimal ctypes view of the HIP runtime that libapus_ghip.so itself links
(/opt/rocm libamdhip64): device buffers, copies, streams and events for the
tests and bench.py.

PyTorch is deliberately not used for device memory here: the installed
torch wheel bundles its own libamdhip64/libhsa-runtime64, and a process that
initialises both runtimes against one device is broken (torch then reports
"No HIP GPUs are available" and the other runtime's results go bad). One
process, one HIP runtime: this one.
"""
import ctypes
import os

import numpy as np

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_hip = None

H2D, D2H, D2D = 1, 2, 3


def hip():
    global _hip
    if _hip is None:
        path = os.path.join(_ROCM, "lib", "libamdhip64.so")
        lib = ctypes.CDLL(path if os.path.exists(path) else "libamdhip64.so")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        sigs = {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, ctypes.c_int],
            "hipMemcpyAsync": [vp, vp, sz, ctypes.c_int, vp],
            "hipMemset": [vp, ctypes.c_int, sz],
            "hipMemsetAsync": [vp, ctypes.c_int, sz, vp],
            "hipDeviceSynchronize": [],
            "hipStreamCreate": [ctypes.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipDeviceGetAttribute": [ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                      ctypes.c_int],
            "hipMemGetInfo": [ctypes.POINTER(sz), ctypes.POINTER(sz)],
            "hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, sz],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.hipGetErrorString.argtypes = [ctypes.c_int]
        lib.hipGetErrorString.restype = ctypes.c_char_p
        _hip = lib
    return _hip


def check(rc, what):
    if rc != 0:
        raise RuntimeError("%s: %s" % (what, hip().hipGetErrorString(rc).decode()))


def device_count():
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(hip().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)),
          "hipMemGetInfo")
    return free.value, total.value


class DevBuf:
    """A hipMalloc'ed device buffer (freed on close/garbage collection)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)),
              "hipMalloc(%d)" % self.nbytes)
        self.ptr = p.value

    @classmethod
    def of(cls, array):
        a = np.ascontiguousarray(array)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    @property
    def vp(self):
        return ctypes.c_void_p(self.ptr)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(hip().hipMemcpy(self.vp, a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                              H2D), "hipMemcpy H2D")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.vp,
                              out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(hip().hipMemset(self.vp, 0, self.nbytes), "hipMemset")

    def close(self):
        if self.ptr:
            hip().hipFree(ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    @property
    def vp(self):
        return ctypes.c_void_p(self.handle)

    def synchronize(self):
        check(hip().hipStreamSynchronize(self.vp), "hipStreamSynchronize")


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream=None):
        check(hip().hipEventRecord(ctypes.c_void_p(self.handle),
                                   stream.vp if stream else None), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(ctypes.c_void_p(self.handle)),
              "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(self.handle),
                                        ctypes.c_void_p(end.handle)),
              "hipEventElapsedTime")
        return ms.value


class Graph:
    """Work enqueued on `stream` between begin() and end(), captured into a
    HIP graph (global capture mode) and instantiated; launch() replays it
    on the stream."""

    def __init__(self, stream):
        self.stream = stream
        self.graph = None
        self.exec = None

    def begin(self):
        check(hip().hipStreamBeginCapture(self.stream.vp, 0), "hipStreamBeginCapture")

    def end(self):
        g = ctypes.c_void_p()
        check(hip().hipStreamEndCapture(self.stream.vp, ctypes.byref(g)),
              "hipStreamEndCapture")
        self.graph = g.value
        e = ctypes.c_void_p()
        check(hip().hipGraphInstantiate(ctypes.byref(e), ctypes.c_void_p(self.graph), None,
                                        None, 0), "hipGraphInstantiate")
        self.exec = e.value

    def launch(self):
        check(hip().hipGraphLaunch(ctypes.c_void_p(self.exec), self.stream.vp),
              "hipGraphLaunch")

    def close(self):
        if self.exec:
            hip().hipGraphExecDestroy(ctypes.c_void_p(self.exec))
            self.exec = None
        if self.graph:
            hip().hipGraphDestroy(ctypes.c_void_p(self.graph))
            self.graph = None
