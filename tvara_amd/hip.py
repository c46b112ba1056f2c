"""Minimal device-memory and event access through the HIP runtime that
libtvara_capi.so itself links (ROCm's libamdhip64.so.7).

Buffers for the device-pointer entry points and HIP-event timing go through
here rather than through a framework: a second HIP runtime in the process
(PyTorch bundles its own) cannot share the GPU with the library's.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _capi

_hip = None
H2D, D2H, D2D = 1, 2, 3


def runtime():
    global _hip
    if _hip is None:
        _capi.lib()  # load the library first so the soname resolves to its runtime
        h = C.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        h.hipEventSynchronize.argtypes = [C.c_void_p]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        h.hipEventDestroy.argtypes = [C.c_void_p]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [C.c_int]
        h.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        h.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        h.hipStreamDestroy.argtypes = [C.c_void_p]
        _hip = h
    return _hip


def check(rc):
    if rc != 0:
        raise RuntimeError(f"HIP error {rc}: {runtime().hipGetErrorString(rc).decode()}")


def synchronize():
    check(runtime().hipDeviceSynchronize())


def copy(dst, src, nbytes):
    """Device-to-device copy of nbytes (the runtime's copy kernel)."""
    check(runtime().hipMemcpy(dst, src, nbytes, D2D))


def device_count():
    n = C.c_int(0)
    rc = runtime().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


class DeviceArray:
    """A block of HBM holding a numpy-shaped array."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(runtime().hipMalloc(C.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(runtime().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D))
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(runtime().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H))
        return out

    def zero(self):
        check(runtime().hipMemset(self.ptr, 0, self.nbytes))

    def free(self):
        if getattr(self, "ptr", None):
            runtime().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        self.free()


class Stream:
    """A HIP stream at the default priority; non_blocking streams do not wait
    for the null stream (hipStreamNonBlocking)."""

    def __init__(self, non_blocking=True):
        p = C.c_void_p()
        check(runtime().hipStreamCreateWithFlags(C.byref(p), 1 if non_blocking else 0))
        self.h = p.value

    def synchronize(self):
        check(runtime().hipStreamSynchronize(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            runtime().hipStreamSynchronize(self.h)
            runtime().hipStreamDestroy(self.h)
            self.h = None


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(runtime().hipEventCreate(C.byref(p)))
        self.h = p.value

    def record(self, stream=None):
        check(runtime().hipEventRecord(self.h, stream))

    def elapsed_ms(self, end):
        check(runtime().hipEventSynchronize(end.h))
        ms = C.c_float()
        check(runtime().hipEventElapsedTime(C.byref(ms), self.h, end.h))
        return ms.value

    def __del__(self):
        if getattr(self, "h", None):
            runtime().hipEventDestroy(self.h)
            self.h = None
