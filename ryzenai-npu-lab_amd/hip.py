"""Minimal ctypes binding of the HIP runtime for torch-free host code.

Device buffers, host<->device copies, stream-ordered events and device
synchronisation -- just what a process needs to drive the C ABI of
liblfm25_hip.so without PyTorch (the benchmark runs this way so that nothing
but the HIP runtime and the decode library is loaded in the measured process).

The runtime is the one liblfm25_hip.so links against (libamdhip64.so.7,
resolved through the library's runpath), so load the decode library first.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

H2D, D2H = 1, 2  # hipMemcpyKind

_rt = None


def runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        _lib.load(bind_torch=False)
        rt = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        for name, args in {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, ctypes.c_int],
            "hipMemset": [vp, ctypes.c_int, sz],
            "hipDeviceSynchronize": [],
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
        }.items():
            fn = getattr(rt, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        rt.hipGetErrorString.restype = ctypes.c_char_p
        rt.hipGetErrorString.argtypes = [ctypes.c_int]
        _rt = rt
    return _rt


def check(err: int, what: str) -> None:
    if err != 0:
        msg = runtime().hipGetErrorString(err).decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}")


def device_count() -> int:
    n = ctypes.c_int(0)
    err = runtime().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def synchronize() -> None:
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Buffer:
    """A device allocation of `nbytes` bytes (freed with the object)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(runtime().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        check(runtime().hipMemcpy(buf.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return buf

    @classmethod
    def zeros(cls, nbytes: int) -> "Buffer":
        buf = cls(nbytes)
        check(runtime().hipMemset(buf.ptr, 0, buf.nbytes), "hipMemset")
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(runtime().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("download larger than the buffer")
        check(runtime().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def __del__(self):
        if getattr(self, "ptr", None) and _rt is not None:
            _rt.hipFree(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(runtime().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream=None) -> None:
        check(runtime().hipEventRecord(self.handle, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(runtime().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        check(runtime().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
              "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        if getattr(self, "handle", None) and _rt is not None:
            _rt.hipEventDestroy(self.handle)
            self.handle = None
