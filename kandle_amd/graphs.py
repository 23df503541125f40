"""HIP graphs of library launches (kh_graph_* in include/kandle_hip.h).

A decode step of a small model is launch-bound: a few hundred short kernels per token, each
dispatched from the host.  Capturing the step once and replaying it with one hipGraphLaunch removes
the per-kernel host work.  The reference has no counterpart; its decode loop dispatches every op
from JavaScript per token (packages/model-utils/src/qwen3/for_causal_lm.ts:475-508).

Rules for code run under `capture()`: it may only enqueue work (no readback, no host-to-device
copy, no synchronisation: those calls fail while a capture is open), and every value that changes
between replays must be read from device memory, not baked in as a launch argument.  Tensors
allocated or freed inside the capture belong to the graph until `dispose()`.
"""
from __future__ import annotations

import ctypes as C
from contextlib import contextmanager

from . import _lib


class HipGraph:
    def __init__(self):
        self._g = None

    @contextmanager
    def capture(self):
        """Record the library launches made inside the `with` block into this graph."""
        if self._g is not None:
            raise RuntimeError("HipGraph: already captured")
        _lib.init_check()
        _lib.call("kh_graph_begin_capture")
        body_ok = False
        try:
            yield self
            body_ok = True
        finally:
            g = C.c_void_p()
            rc = _lib.load().kh_graph_end_capture(C.byref(g))
            if body_ok:
                _lib.check(rc, "kh_graph_end_capture")
                self._g = g
            elif rc == 0:  # the body raised: drop the partial graph, re-raise the body's error
                _lib.load().kh_graph_destroy(g)

    @property
    def captured(self) -> bool:
        return self._g is not None

    def replay(self) -> None:
        if self._g is None:
            raise RuntimeError("HipGraph: nothing captured")
        _lib.call("kh_graph_launch", self._g)

    def dispose(self) -> None:
        if self._g is not None:
            _lib.call("kh_graph_destroy", self._g)
            self._g = None
