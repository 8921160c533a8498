"""Device memory, streams and events for tests and benchmarks.

Binds the HIP runtime that libpai_hip.so itself links (libamdhip64.so.7,
resolved through the already-loaded library), so buffers, streams and
events live in the same runtime as the kernels. torch is deliberately not
used for device memory: its wheel bundles a second HIP/HSA runtime with
the same soname, and a process that initialises both sees torch's device
init fail ("No HIP GPUs are available").
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import lib

_hip = None

H2D, D2H, D2D = 1, 2, 3  # hipMemcpyKind


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        lib()  # loads libpai_hip.so and, through it, its HIP runtime
        h = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        sigs = {
            "hipMalloc": [C.POINTER(vp), C.c_size_t],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, C.c_size_t, C.c_int],
            "hipMemcpyAsync": [vp, vp, C.c_size_t, C.c_int, vp],
            "hipMemsetAsync": [vp, C.c_int, C.c_size_t, vp],
            "hipDeviceSynchronize": [],
            "hipStreamCreate": [C.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [C.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [C.POINTER(C.c_float), vp, vp],
            "hipGetLastError": [],
            "hipStreamBeginCapture": [vp, C.c_int],
            "hipStreamEndCapture": [vp, C.POINTER(vp)],
            "hipGraphInstantiate": [C.POINTER(vp), vp, vp, C.c_char_p, C.c_size_t],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }
        for name, args in sigs.items():
            fn = getattr(h, name)
            fn.restype = C.c_int
            fn.argtypes = args
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [C.c_int]
        _hip = h
    return _hip


def hip_check(err: int, where: str) -> None:
    if err != 0:
        raise RuntimeError(f"{where}: {hip().hipGetErrorString(err).decode()} ({err})")


class DeviceBuffer:
    """A raw device allocation (hipMalloc) of `nbytes`."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self._p = C.c_void_p()
        hip_check(hip().hipMalloc(C.byref(self._p), max(self.nbytes, 1)), "hipMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    @property
    def ptr(self) -> int:
        return self._p.value

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, shape, dtype=np.float32, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, D2H),
                  "hipMemcpy D2H")
        return out

    def free(self) -> None:
        if self._p.value:
            hip_check(hip().hipFree(self._p), "hipFree")
            self._p = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A default-priority HIP stream."""

    def __init__(self):
        self._s = C.c_void_p()
        hip_check(hip().hipStreamCreate(C.byref(self._s)), "hipStreamCreate")

    @property
    def handle(self) -> int:
        return self._s.value

    def synchronize(self) -> None:
        hip_check(hip().hipStreamSynchronize(self._s), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self._s.value:
            hip().hipStreamDestroy(self._s)
            self._s = C.c_void_p()


class Event:
    def __init__(self):
        self._e = C.c_void_p()
        hip_check(hip().hipEventCreate(C.byref(self._e)), "hipEventCreate")

    def record(self, stream: Stream | None) -> None:
        hip_check(hip().hipEventRecord(self._e, stream.handle if stream else None),
                  "hipEventRecord")

    def synchronize(self) -> None:
        hip_check(hip().hipEventSynchronize(self._e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        t = C.c_float()
        hip_check(hip().hipEventElapsedTime(C.byref(t), self._e, end._e), "hipEventElapsedTime")
        return float(t.value)

    def destroy(self) -> None:
        if self._e.value:
            hip().hipEventDestroy(self._e)
            self._e = C.c_void_p()


def synchronize() -> None:
    hip_check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Graph:
    """A HIP graph captured from the work `fn(stream_handle)` enqueues on a
    stream (hipStreamBeginCapture ... hipStreamEndCapture), instantiated
    once and replayed with one host call."""

    def __init__(self, stream: Stream, fn):
        g = C.c_void_p()
        hip_check(hip().hipStreamBeginCapture(stream._s, 1), "hipStreamBeginCapture")  # thread-local
        try:
            fn(stream.handle)
        finally:
            hip_check(hip().hipStreamEndCapture(stream._s, C.byref(g)), "hipStreamEndCapture")
        self._g = g
        self._e = C.c_void_p()
        hip_check(hip().hipGraphInstantiate(C.byref(self._e), g, None, None, 0),
                  "hipGraphInstantiate")

    def launch(self, stream: Stream) -> None:
        hip_check(hip().hipGraphLaunch(self._e, stream._s), "hipGraphLaunch")

    def destroy(self) -> None:
        if self._e.value:
            hip().hipGraphExecDestroy(self._e)
            self._e = C.c_void_p()
        if self._g.value:
            hip().hipGraphDestroy(self._g)
            self._g = C.c_void_p()
