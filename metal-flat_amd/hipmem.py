# SPDX-License-Identifier: Apache-2.0
"""Minimal device-memory plumbing over the HIP runtime that libmflat.so itself
links (libamdhip64.so.7, resolved through the already-loaded library), for
callers and benchmarks that want device-resident inputs without a second
framework.

torch wheels bundle their own copy of the HIP and HSA runtimes; a process that
loads libmflat.so first and then initialises torch's GPU backend ends up with two
runtimes competing for the device. When torch must share the process, import it
and touch its GPU backend BEFORE loading libmflat.so: the loader then binds the
library to torch's copy (same SONAME), and there is a single runtime.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_size_t, c_void_p, c_float

import numpy as np

import mflat

_hip = None
H2D, D2H, D2D = 1, 2, 3


def hip():
    global _hip
    if _hip is None:
        mflat.load()
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [ctypes.POINTER(c_void_p), c_size_t]
        h.hipFree.argtypes = [c_void_p]
        h.hipMemcpy.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        h.hipMemset.argtypes = [c_void_p, c_int, c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipGetDeviceCount.argtypes = [ctypes.POINTER(c_int)]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [c_int]
        h.hipStreamCreate.argtypes = [ctypes.POINTER(c_void_p)]
        h.hipStreamDestroy.argtypes = [c_void_p]
        h.hipStreamSynchronize.argtypes = [c_void_p]
        h.hipEventCreate.argtypes = [ctypes.POINTER(c_void_p)]
        h.hipEventDestroy.argtypes = [c_void_p]
        h.hipEventRecord.argtypes = [c_void_p, c_void_p]
        h.hipEventSynchronize.argtypes = [c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(c_float), c_void_p, c_void_p]
        _hip = h
    return _hip


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error {rc} ({hip().hipGetErrorString(rc).decode()})")


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceArray:
    """A contiguous device allocation with a numpy-like shape/dtype."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = c_void_p()
        check(hip().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)), "hipMalloc")

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(hip().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value: int) -> None:
        check(hip().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    def data_ptr(self) -> int:
        return self.ptr.value

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.handle = c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    @property
    def cuda_stream(self) -> int:
        return self.handle.value or 0

    def synchronize(self) -> None:
        check(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(self.handle)
            self.handle = c_void_p()
