"""Device buffers, copies and events through the HIP runtime that libeakv.so
itself links (ctypes on libamdhip64.so.7), for the tests and the benchmark.

Loading libeakv first guarantees that this module and the library talk to the
same runtime instance, so device pointers pass freely between them.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib as _eakv_lib

_vp = C.c_void_p
_HIP = None

H2D, D2H, D2D = 1, 2, 3


def hip():
    global _HIP
    if _HIP is None:
        _eakv_lib()
        h = C.CDLL("libamdhip64.so.7")
        sig = {
            "hipMalloc": [C.POINTER(_vp), C.c_size_t],
            "hipFree": [_vp],
            "hipMemcpy": [_vp, _vp, C.c_size_t, C.c_int],
            "hipMemcpyAsync": [_vp, _vp, C.c_size_t, C.c_int, _vp],
            "hipMemsetAsync": [_vp, C.c_int, C.c_size_t, _vp],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [_vp],
            "hipStreamCreateWithFlags": [C.POINTER(_vp), C.c_uint],
            "hipStreamDestroy": [_vp],
            "hipEventCreate": [C.POINTER(_vp)],
            "hipEventDestroy": [_vp],
            "hipEventRecord": [_vp, _vp],
            "hipEventSynchronize": [_vp],
            "hipEventElapsedTime": [C.POINTER(C.c_float), _vp, _vp],
            "hipGetDeviceCount": [C.POINTER(C.c_int)],
            "hipMemGetInfo": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)],
            "hipGetErrorString": [C.c_int],
        }
        for n, a in sig.items():
            f = getattr(h, n)
            f.argtypes = a
            f.restype = C.c_int
        h.hipGetErrorString.restype = C.c_char_p
        _HIP = h
    return _HIP


def check(err, what="hip"):
    if err != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(err).decode()} ({err})")


def device_count():
    n = C.c_int(0)
    if hip().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def mem_info():
    f, t = C.c_size_t(), C.c_size_t()
    check(hip().hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
    return f.value, t.value


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceArray:
    """A hipMalloc'd buffer with a numpy shape/dtype."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = _vp()
        check(hip().hipMalloc(C.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_host(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a, self.dtype)
        assert a.nbytes == self.nbytes
        check(hip().hipMemcpy(self.ptr, a.ctypes.data_as(_vp), self.nbytes, H2D), "H2D")

    def download(self):
        a = np.empty(self.shape, self.dtype)
        check(hip().hipMemcpy(a.ctypes.data_as(_vp), self.ptr, self.nbytes, D2H), "D2H")
        return a

    def zero(self, stream=None):
        check(hip().hipMemsetAsync(self.ptr, 0, self.nbytes, stream), "memset")

    def offset(self, nbytes):
        return self.ptr + nbytes

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream at the default priority."""

    def __init__(self):
        st = _vp()
        check(hip().hipStreamCreateWithFlags(C.byref(st), 1), "hipStreamCreateWithFlags")
        self.s = st.value

    def synchronize(self):
        check(hip().hipStreamSynchronize(self.s), "hipStreamSynchronize")

    def __del__(self):
        try:
            hip().hipStreamDestroy(self.s)
        except Exception:
            pass


class Event:
    def __init__(self):
        e = _vp()
        check(hip().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream=None):
        check(hip().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, later):
        ms = C.c_float()
        check(hip().hipEventElapsedTime(C.byref(ms), self.e, later.e), "elapsed")
        return ms.value

    def __del__(self):
        try:
            hip().hipEventDestroy(self.e)
        except Exception:
            pass
