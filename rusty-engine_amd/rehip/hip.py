"""Minimal ctypes plumbing over the HIP runtime that librehip.so links (libamdhip64.so.7 from
/opt/rocm): device buffers, copies, streams and events for the device-pointer entry points,
the benchmark and the tests.

torch is deliberately not used in processes that load librehip: torch bundles its own HIP
runtime under the same soname, and two HIP runtimes in one process do not initialise.
"""
from __future__ import annotations

import ctypes as C
import ctypes  # noqa: F401  (re-exported for callers building raw calls)

import numpy as np

from . import lib as _rehip_lib

_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        _rehip_lib()                    # loads libamdhip64.so.7 through librehip's RUNPATH
        H = C.CDLL("libamdhip64.so.7")
        H.hipGetErrorString.restype = C.c_char_p
        H.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        H.hipFree.argtypes = [C.c_void_p]
        H.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        H.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        H.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        H.hipDeviceSynchronize.argtypes = []
        H.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        H.hipStreamDestroy.argtypes = [C.c_void_p]
        H.hipStreamSynchronize.argtypes = [C.c_void_p]
        H.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        H.hipEventDestroy.argtypes = [C.c_void_p]
        H.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        H.hipEventSynchronize.argtypes = [C.c_void_p]
        H.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        H.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        H.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        H.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        H.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
        H.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        H.hipGraphExecDestroy.argtypes = [C.c_void_p]
        H.hipGraphDestroy.argtypes = [C.c_void_p]
        _hip = H
    return _hip


H2D, D2H, D2D = 1, 2, 3


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"HIP error {rc}: {hip().hipGetErrorString(rc).decode()}")


def device_count() -> int:
    n = C.c_int(0)
    rc = hip().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


class DeviceBuffer:
    """Owned device allocation of `nbytes` bytes."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(hip().hipMalloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(hip().hipMemcpy(C.c_void_p(self.ptr), a.ctypes.data, a.nbytes, H2D))

    def download(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        itemsize = np.dtype(dtype).itemsize
        n = self.nbytes // itemsize if count is None else count
        out = np.empty(n, dtype)
        check(hip().hipMemcpy(out.ctypes.data, C.c_void_p(self.ptr), n * itemsize, D2H))
        return out

    def zero(self) -> None:
        check(hip().hipMemset(C.c_void_p(self.ptr), 0, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        check(hip().hipStreamCreate(C.byref(s)))
        self.handle = s.value

    def synchronize(self) -> None:
        check(hip().hipStreamSynchronize(C.c_void_p(self.handle)))

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(C.c_void_p(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(hip().hipEventCreate(C.byref(e)))
        self.ev = e.value

    def record(self, stream: Stream | None = None) -> None:
        check(hip().hipEventRecord(C.c_void_p(self.ev), C.c_void_p(stream.handle if stream else None)))

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(C.c_void_p(self.ev)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(hip().hipEventElapsedTime(C.byref(ms), C.c_void_p(self.ev), C.c_void_p(end.ev)))
        return ms.value


class Graph:
    """A HIP graph captured from the calls `fn()` makes on `stream` (stream capture), then
    instantiated for replay. Captured work must not contain memset nodes."""

    def __init__(self, stream: Stream, fn):
        H = hip()
        check(H.hipStreamBeginCapture(C.c_void_p(stream.handle), 0))   # hipStreamCaptureModeGlobal
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = H.hipStreamEndCapture(C.c_void_p(stream.handle), C.byref(g))
        check(rc)
        self.graph = g.value
        ex = C.c_void_p()
        check(H.hipGraphInstantiate(C.byref(ex), C.c_void_p(self.graph), None, None, 0))
        self.exec = ex.value
        self.stream = stream

    def launch(self) -> None:
        check(hip().hipGraphLaunch(C.c_void_p(self.exec), C.c_void_p(self.stream.handle)))

    def destroy(self) -> None:
        if self.exec:
            hip().hipGraphExecDestroy(C.c_void_p(self.exec))
            hip().hipGraphDestroy(C.c_void_p(self.graph))
            self.exec = self.graph = None


def synchronize() -> None:
    check(hip().hipDeviceSynchronize())
