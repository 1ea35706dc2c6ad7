"""Stream capture of the context's launches into a HIP graph, through the HIP
runtime the library itself is linked against (libamdhip64.so.7).

The library enqueues on whatever stream ehip_set_stream gave it; a caller
that captures that stream records the per-layer step launches (kernels only)
into a graph it can replay. This module is that caller's side in a few ctypes
calls, for the tests and bench.py. PyTorch users can do the same with
torch.cuda.CUDAGraph on a torch stream, provided torch's HIP runtime is the
one the library uses (torch imported before the library is loaded).
"""
from __future__ import annotations

import ctypes as C

from . import lib

_hip = None
_CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal


def hip():
    """The HIP runtime already loaded by libehip.so (same instance)."""
    global _hip
    if _hip is None:
        lib()  # loads libehip.so and with it libamdhip64.so.7
        h = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        h.hipStreamCreateWithFlags.argtypes = [C.POINTER(vp), C.c_uint]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        h.hipGraphExecUpdate.argtypes = [vp, vp, C.POINTER(vp), C.POINTER(C.c_int)]
        _hip = h
    return _hip


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


class Stream:
    """A non-blocking HIP stream (default priority)."""

    def __init__(self):
        self.h = C.c_void_p()
        _ok(hip().hipStreamCreateWithFlags(C.byref(self.h), 1), "hipStreamCreateWithFlags")

    def synchronize(self):
        _ok(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def close(self):
        if self.h:
            hip().hipStreamDestroy(self.h)
            self.h = C.c_void_p()


class Graph:
    """capture(stream, fn): records what fn enqueues on stream; replay(stream)."""

    def __init__(self):
        self.graph = C.c_void_p()
        self.exec = C.c_void_p()

    def capture(self, stream: Stream, fn):
        _ok(hip().hipStreamBeginCapture(stream.h, _CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            _ok(hip().hipStreamEndCapture(stream.h, C.byref(self.graph)), "hipStreamEndCapture")
        _ok(hip().hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0),
            "hipGraphInstantiate")
        return self

    def update(self, stream: Stream, fn):
        """Re-capture what fn enqueues (the same launch sequence for a new step
        plan) and write its kernel parameters into the instantiated graph
        (hipGraphExecUpdate): no re-instantiation. Raises if the launch
        topology changed (then capture() a new graph instead)."""
        g = C.c_void_p()
        _ok(hip().hipStreamBeginCapture(stream.h, _CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            _ok(hip().hipStreamEndCapture(stream.h, C.byref(g)), "hipStreamEndCapture")
        err_node, result = C.c_void_p(), C.c_int(-1)
        rc = hip().hipGraphExecUpdate(self.exec, g, C.byref(err_node), C.byref(result))
        if rc != 0:
            hip().hipGraphDestroy(g)
            raise RuntimeError(f"hipGraphExecUpdate failed: hipError {rc}, update result "
                               f"{result.value}")
        hip().hipGraphDestroy(self.graph)
        self.graph = g
        return self

    def replay(self, stream: Stream):
        _ok(hip().hipGraphLaunch(self.exec, stream.h), "hipGraphLaunch")

    def close(self):
        if self.exec:
            hip().hipGraphExecDestroy(self.exec)
            self.exec = C.c_void_p()
        if self.graph:
            hip().hipGraphDestroy(self.graph)
            self.graph = C.c_void_p()
