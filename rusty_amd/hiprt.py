"""Minimal ctypes access to the HIP runtime that librusty_hip.so links.

Timing (hipEvent*), extra streams (default priority) and stream capture into
HIP graphs (hipStreamBeginCapture ... hipGraphLaunch) for the benchmark and
the graph-replay tests.  The
runtime is the same ``libamdhip64.so.7`` instance the library loaded.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_float, c_int, c_void_p

from . import _lib

_hip = None
HIP_STREAM_CAPTURE_MODE_GLOBAL = 0
HIP_STREAM_CAPTURE_MODE_THREAD_LOCAL = 1


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _lib.lib()  # loads libamdhip64.so.7 as a dependency first
        h = ctypes.CDLL("libamdhip64.so.7")
        P = c_void_p
        sig = {
            "hipEventCreate": [POINTER(c_void_p)],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [POINTER(c_float), P, P],
            "hipEventDestroy": [P],
            "hipStreamBeginCapture": [P, c_int],
            "hipStreamEndCapture": [P, POINTER(c_void_p)],
            "hipGraphInstantiate": [POINTER(c_void_p), P, P, P, ctypes.c_size_t],
            "hipGraphLaunch": [P, P],
            "hipGraphExecDestroy": [P],
            "hipGraphDestroy": [P],
            "hipStreamSynchronize": [P],
            "hipStreamCreateWithFlags": [POINTER(c_void_p), ctypes.c_uint],
            "hipStreamDestroy": [P],
            "hipDeviceSynchronize": [],
            "hipGetErrorString": [c_int],
        }
        for name, args in sig.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = ctypes.c_char_p if name == "hipGetErrorString" else c_int
        _hip = h
    return _hip


def _ok(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(err).decode()} ({err})")


class Event:
    def __init__(self):
        self.h = c_void_p()
        _ok(hip().hipEventCreate(byref(self.h)), "hipEventCreate")

    def record(self, stream) -> None:
        _ok(hip().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self) -> None:
        _ok(hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        _ok(hip().hipEventElapsedTime(byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.h:
                hip().hipEventDestroy(self.h)
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream of default priority (streams of other
    priorities are not used)."""

    def __init__(self):
        self.h = c_void_p()
        _ok(hip().hipStreamCreateWithFlags(byref(self.h), 1), "hipStreamCreateWithFlags")

    def synchronize(self) -> None:
        _ok(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.h:
                hip().hipStreamSynchronize(self.h)
                hip().hipStreamDestroy(self.h)
        except Exception:
            pass


class Graph:
    """Captures the work a callable enqueues on ``stream`` into a HIP graph."""

    def __init__(self, stream, enqueue):
        h = hip()
        _ok(h.hipStreamBeginCapture(stream, HIP_STREAM_CAPTURE_MODE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            enqueue()
        finally:
            g = c_void_p()
            err = h.hipStreamEndCapture(stream, byref(g))
        _ok(err, "hipStreamEndCapture")
        self.graph = g
        self.exec = c_void_p()
        _ok(h.hipGraphInstantiate(byref(self.exec), g, None, None, 0), "hipGraphInstantiate")
        self.stream = stream

    def launch(self) -> None:
        _ok(hip().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        try:
            hip().hipGraphExecDestroy(self.exec)
            hip().hipGraphDestroy(self.graph)
        except Exception:
            pass
