"""Minimal ctypes binding of the HIP runtime used by libwisp_amd.so.

Device memory, streams and events for the tests, the smoke check and the
benchmark. It binds the same libamdhip64 instance the library links, so
pointers and streams are shared with it. torch is deliberately not used:
it bundles its own HIP runtime under the same soname.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_float, c_int, c_size_t, c_uint, c_void_p

import numpy as np

_HIP = None

hipMemcpyHostToDevice = 1
hipMemcpyDeviceToHost = 2
hipMemcpyDeviceToDevice = 3


class HipError(RuntimeError):
    pass


def runtime():
    global _HIP
    if _HIP is None:
        from . import _lib  # the product library pulls in libamdhip64 first
        _lib.lib()
        h = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [c_int]
        for name, args in {
            "hipMalloc": [POINTER(c_void_p), c_size_t],
            "hipFree": [c_void_p],
            "hipHostMalloc": [POINTER(c_void_p), c_size_t, c_uint],
            "hipHostFree": [c_void_p],
            "hipMemcpy": [c_void_p, c_void_p, c_size_t, c_int],
            "hipMemcpyAsync": [c_void_p, c_void_p, c_size_t, c_int, c_void_p],
            "hipMemset": [c_void_p, c_int, c_size_t],
            "hipMemsetAsync": [c_void_p, c_int, c_size_t, c_void_p],
            "hipStreamCreate": [POINTER(c_void_p)],
            "hipStreamDestroy": [c_void_p],
            "hipStreamSynchronize": [c_void_p],
            "hipDeviceSynchronize": [],
            "hipEventCreate": [POINTER(c_void_p)],
            "hipEventDestroy": [c_void_p],
            "hipEventRecord": [c_void_p, c_void_p],
            "hipEventSynchronize": [c_void_p],
            "hipEventElapsedTime": [POINTER(c_float), c_void_p, c_void_p],
            "hipGetDeviceCount": [POINTER(c_int)],
            "hipSetDevice": [c_int],
            "hipGetLastError": [],
            "hipMemGetInfo": [POINTER(c_size_t), POINTER(c_size_t)],
            "hipStreamBeginCapture": [c_void_p, c_int],
            "hipStreamEndCapture": [c_void_p, POINTER(c_void_p)],
            "hipGraphInstantiate": [POINTER(c_void_p), c_void_p, c_void_p, c_void_p, c_size_t],
            "hipGraphLaunch": [c_void_p, c_void_p],
            "hipGraphExecDestroy": [c_void_p],
            "hipGraphDestroy": [c_void_p],
        }.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = c_int
        _HIP = h
    return _HIP


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = runtime().hipGetErrorString(rc).decode()
        raise HipError(f"{what}: HIP error {rc} ({msg})")


def device_count() -> int:
    n = c_int(0)
    rc = runtime().hipGetDeviceCount(byref(n))
    return n.value if rc == 0 else 0


def synchronize() -> None:
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info() -> tuple[int, int]:
    free, total = c_size_t(0), c_size_t(0)
    check(runtime().hipMemGetInfo(byref(free), byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """Owned device allocation; `ptr` is the raw device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(runtime().hipMalloc(byref(p), max(self.nbytes, 1)), f"hipMalloc({nbytes})")
        self._p = p

    @property
    def ptr(self) -> int:
        return self._p.value or 0

    def __int__(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self._p is not None and self._p.value:
            runtime().hipFree(self._p)
        self._p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr: np.ndarray, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, (offset, a.nbytes, self.nbytes)
        check(runtime().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes,
                                  hipMemcpyHostToDevice), "H2D")
        return self

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(runtime().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes,
                                  hipMemcpyDeviceToHost), "D2H")
        return out

    def zero(self) -> "DeviceBuffer":
        check(runtime().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")
        return self


def to_device(arr: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(arr)
    return DeviceBuffer(a.nbytes).upload(a)


class PinnedBuffer:
    """Page-locked host allocation (hipHostMalloc) viewed as a numpy array."""

    def __init__(self, nbytes: int):
        p = c_void_p()
        check(runtime().hipHostMalloc(byref(p), max(int(nbytes), 1), 0), f"hipHostMalloc({nbytes})")
        self._p = p
        self.nbytes = int(nbytes)
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(p.value))

    @property
    def ptr(self) -> int:
        return self._p.value or 0

    def free(self) -> None:
        if self._p is not None and self._p.value:
            runtime().hipHostFree(self._p)
        self._p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = c_void_p()
        check(runtime().hipStreamCreate(byref(s)), "hipStreamCreate")
        self._s = s

    @property
    def handle(self) -> int:
        return self._s.value or 0

    def synchronize(self) -> None:
        check(runtime().hipStreamSynchronize(self._s), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self._s is not None and self._s.value:
                runtime().hipStreamDestroy(self._s)
        except Exception:
            pass


class Event:
    def __init__(self):
        e = c_void_p()
        check(runtime().hipEventCreate(byref(e)), "hipEventCreate")
        self._e = e

    @property
    def handle(self) -> int:
        return self._e.value or 0

    def record(self, stream: int = 0) -> None:
        check(runtime().hipEventRecord(self._e, c_void_p(stream)), "hipEventRecord")

    def synchronize(self) -> None:
        check(runtime().hipEventSynchronize(self._e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        t = c_float(0)
        check(runtime().hipEventElapsedTime(byref(t), self._e, end._e), "hipEventElapsedTime")
        return float(t.value)

    def __del__(self):
        try:
            if self._e is not None and self._e.value:
                runtime().hipEventDestroy(self._e)
        except Exception:
            pass


hipStreamCaptureModeThreadLocal = 1


class Graph:
    """A HIP graph captured from the launches `fn()` makes on `stream`,
    instantiated for replay with launch()."""

    def __init__(self, stream: Stream, fn):
        rt = runtime()
        check(rt.hipStreamBeginCapture(c_void_p(stream.handle), hipStreamCaptureModeThreadLocal),
              "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = c_void_p()
            rc = rt.hipStreamEndCapture(c_void_p(stream.handle), byref(g))
        check(rc, "hipStreamEndCapture")
        self._g = g
        ex = c_void_p()
        check(rt.hipGraphInstantiate(byref(ex), g, None, None, 0), "hipGraphInstantiate")
        self._ex = ex

    def launch(self, stream: Stream) -> None:
        check(runtime().hipGraphLaunch(self._ex, c_void_p(stream.handle)), "hipGraphLaunch")

    def __del__(self):
        try:
            if self._ex is not None and self._ex.value:
                runtime().hipGraphExecDestroy(self._ex)
            if self._g is not None and self._g.value:
                runtime().hipGraphDestroy(self._g)
        except Exception:
            pass
