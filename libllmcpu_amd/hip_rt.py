"""A few HIP runtime calls through ctypes (device memory, copies, events,
graphs), for the benchmark and the tests; the attention op itself is in
libnnc_hip.so."""
from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        h = C.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        h.hipEventSynchronize.argtypes = [C.c_void_p]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        h.hipEventDestroy.argtypes = [C.c_void_p]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipDeviceGetAttribute.argtypes = [C.POINTER(C.c_int), C.c_int, C.c_int]
        h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        h.hipGraphExecDestroy.argtypes = [C.c_void_p]
        h.hipGraphDestroy.argtypes = [C.c_void_p]
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        _hip = h
    return _hip


def check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(err).decode()}")


def malloc(nbytes: int) -> int:
    p = C.c_void_p()
    check(hip().hipMalloc(C.byref(p), nbytes), "hipMalloc")
    return p.value


def free(ptr: int) -> None:
    if ptr:
        check(hip().hipFree(ptr), "hipFree")


def to_device(ptr: int, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a)
    check(hip().hipMemcpy(ptr, a.ctypes.data, a.nbytes, 1), "hipMemcpy H2D")


def to_host(a: np.ndarray, ptr: int) -> np.ndarray:
    check(hip().hipMemcpy(a.ctypes.data, ptr, a.nbytes, 2), "hipMemcpy D2H")
    return a


def sync() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


def device_count() -> int:
    n = C.c_int(0)
    return n.value if hip().hipGetDeviceCount(C.byref(n)) == 0 else 0


def attribute(attr: int, device: int = 0) -> int:
    v = C.c_int(0)
    check(hip().hipDeviceGetAttribute(C.byref(v), attr, device), "hipDeviceGetAttribute")
    return v.value


class Event:
    """A HIP event recorded on a given stream (a hipStream_t address)."""

    def __init__(self):
        self.e = C.c_void_p()
        check(hip().hipEventCreate(C.byref(self.e)), "hipEventCreate")

    def record(self, stream: int) -> None:
        check(hip().hipEventRecord(self.e, stream or None), "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(self.e), "hipEventSynchronize")

    def ms_since(self, start: "Event") -> float:
        ms = C.c_float(0.0)
        check(hip().hipEventElapsedTime(C.byref(ms), start.e, self.e), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            hip().hipEventDestroy(self.e)
        except Exception:
            pass


class Graph:
    """The kernel launches `fn()` issues on `stream`, captured once into a HIP
    graph (thread-local capture: any allocation or synchronisation inside
    fn() fails the capture) and replayed with launch(). fn() must not record
    memset nodes."""

    def __init__(self, stream: int, fn):
        h = hip()
        check(h.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")
        g = C.c_void_p()
        try:
            fn()
        finally:
            err = h.hipStreamEndCapture(stream, C.byref(g))
        check(err, "hipStreamEndCapture")
        self.graph = g
        self.exec = C.c_void_p()
        check(h.hipGraphInstantiate(C.byref(self.exec), g, None, None, 0), "hipGraphInstantiate")

    def launch(self, stream: int) -> None:
        check(hip().hipGraphLaunch(self.exec, stream), "hipGraphLaunch")

    def close(self) -> None:
        if self.exec:
            hip().hipGraphExecDestroy(self.exec)
            self.exec = C.c_void_p()
        if self.graph:
            hip().hipGraphDestroy(self.graph)
            self.graph = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
