"""Minimal ctypes access to the HIP runtime: device buffers, streams and events.

Used to hold inputs resident in HBM and to time the `_dev` entry points of the head
library with HIP events on the stream the kernels run on.  Plumbing only.
"""
import ctypes
import os

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        _hip = ctypes.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        _hip.hipGetErrorString.restype = ctypes.c_char_p
        _hip.hipGetErrorString.argtypes = [ctypes.c_int]
    return _hip


class HipError(RuntimeError):
    pass


def check(rc, what):
    if rc != 0:
        raise HipError(f"{what}: {hip().hipGetErrorString(rc).decode()} ({rc})")


H2D, D2H, D2D = 1, 2, 3


def device_count():
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def device_name(dev=0):
    # hipDeviceProp_t is large; read gcnArchName through hipDeviceGetAttribute-free path.
    buf = ctypes.create_string_buffer(4096)
    check(hip().hipGetDevicePropertiesR0600(buf, dev), "hipGetDeviceProperties")
    name = buf.raw[:256].split(b"\0", 1)[0].decode(errors="replace")
    return name


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(max(self.nbytes, 1))), "hipMalloc")

    @classmethod
    def from_numpy(cls, arr):
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        if d.nbytes:
            check(hip().hipMemcpy(d.ptr, arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(d.nbytes), H2D),
                  "hipMemcpy H2D")
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, ctypes.c_size_t(self.nbytes), D2H),
                  "hipMemcpy D2H")
        return out

    def fill_bytes(self, value=0):
        check(hip().hipMemset(self.ptr, ctypes.c_int(value), ctypes.c_size_t(max(self.nbytes, 1))), "hipMemset")

    @property
    def p(self):
        return self.ptr

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.h = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(self.h)), "hipStreamCreate")

    def synchronize(self):
        check(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.h:
                hip().hipStreamDestroy(self.h)
        except Exception:
            pass


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream):
        check(hip().hipEventRecord(self.h, stream.h if stream is not None else None), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.h:
                hip().hipEventDestroy(self.h)
        except Exception:
            pass
