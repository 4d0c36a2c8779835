"""Minimal ctypes view of the HIP runtime for timing and graph replay.

Used by callers that drive the provider and want device-side timing on the
provider's own stream (HIP events) or to capture a compiled step into a HIP
graph and replay it.  Loads the same libamdhip64 the provider links.
"""
from __future__ import annotations

import ctypes as C
import os

_hip = None


def lib() -> C.CDLL:
    global _hip
    if _hip is None:
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        for name in ("libamdhip64.so", os.path.join(rocm, "lib", "libamdhip64.so")):
            try:
                _hip = C.CDLL(name)
                break
            except OSError:
                continue
        if _hip is None:
            raise RuntimeError("libamdhip64.so not found")
        h = _hip
        for fn, args in {
            "hipEventCreate": [C.POINTER(C.c_void_p)],
            "hipEventDestroy": [C.c_void_p],
            "hipEventRecord": [C.c_void_p, C.c_void_p],
            "hipEventSynchronize": [C.c_void_p],
            "hipEventElapsedTime": [C.POINTER(C.c_float), C.c_void_p, C.c_void_p],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [C.c_void_p],
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
            "hipGetErrorString": [C.c_int],
        }.items():
            f = getattr(h, fn)
            f.argtypes = args
            f.restype = C.c_char_p if fn == "hipGetErrorString" else C.c_int
    return _hip


def check(err: int, where: str) -> None:
    if err != 0:
        raise RuntimeError(f"{where}: hip error {err} ({lib().hipGetErrorString(err).decode()})")


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(lib().hipEventCreate(C.byref(self.h)), "hipEventCreate")

    def record(self, stream: int) -> None:
        check(lib().hipEventRecord(self.h, C.c_void_p(stream)), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.h:
                lib().hipEventDestroy(self.h)
        except Exception:
            pass


def device_synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Graph:
    """Capture everything enqueued on `stream` by `fn()` into a graph."""

    CAPTURE_GLOBAL = 0

    def __init__(self, stream: int, fn):
        self.stream = C.c_void_p(stream)
        graph = C.c_void_p()
        check(lib().hipStreamBeginCapture(self.stream, self.CAPTURE_GLOBAL), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            err = lib().hipStreamEndCapture(self.stream, C.byref(graph))
        check(err, "hipStreamEndCapture")
        self.graph = graph
        self.exec = C.c_void_p()
        check(lib().hipGraphInstantiate(C.byref(self.exec), graph, None, None, 0), "hipGraphInstantiate")

    def launch(self) -> None:
        check(lib().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        try:
            lib().hipGraphExecDestroy(self.exec)
            lib().hipGraphDestroy(self.graph)
        except Exception:
            pass
