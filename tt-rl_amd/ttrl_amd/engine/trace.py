"""hipGraph capture and replay (replaces ttrl/engine/trace.py:56-126).

Capture is a callback API for the reference's reason: every path out of the
recording region goes through this module's own try, so a failed capture is
always ended and discarded and the stream never stays in capture mode.
"""

from __future__ import annotations

import ctypes as C
from typing import Callable, TypeVar

from ttrl_amd import _lib

__all__ = ["HOST_READ_DURING_CAPTURE", "CapturedTrace", "TraceCaptureError", "capture"]

HOST_READ_DURING_CAPTURE = "not supported during graph capture"

R = TypeVar("R")


class TraceCaptureError(RuntimeError):
    """Capture failed.  There is no eager fallback."""


class CapturedTrace:
    """One instantiated graph, replayable until closed."""

    __slots__ = ("device", "_graph", "pool")

    def __init__(self, device, graph: C.c_void_p, pool: int | None = None):
        self.device = device
        self._graph = graph
        self.pool = pool

    @property
    def live(self) -> bool:
        return self._graph is not None

    @property
    def nodes(self) -> int:
        n = C.c_size_t(0)
        _lib.check(_lib.lib().ttrl_graph_nodes(self._graph, C.byref(n)), "ttrl_graph_nodes")
        return int(n.value)

    def replay(self, *, cfg=None, blocking: bool | None = None) -> None:
        if self._graph is None:
            raise RuntimeError("replay() on a closed CapturedTrace")
        self.device.call("ttrl_graph_launch", self._graph)
        if blocking:
            self.device.synchronize()

    def set_direct(self, on: bool = True) -> None:
        """Replay the graph's kernels as individual launches (ttrl_graph_set_direct):
        cheaper than one graph launch for a few kernels replayed once per host step."""
        if self._graph is None:
            raise RuntimeError("set_direct() on a closed CapturedTrace")
        _lib.check(_lib.lib().ttrl_graph_set_direct(self._graph, int(bool(on))), "ttrl_graph_set_direct")

    def replay_n(self, n: int) -> None:
        if self._graph is None:
            raise RuntimeError("replay_n() on a closed CapturedTrace")
        self.device.call("ttrl_graph_launch_n", self._graph, int(n))

    def close(self) -> None:
        if self._graph is None:
            return
        graph, self._graph = self._graph, None
        if not self.device.closed:
            self.device.synchronize()
            _lib.lib().ttrl_graph_destroy(graph)

    def __enter__(self) -> "CapturedTrace":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def capture(device, record: Callable[[], R]) -> tuple[CapturedTrace, R]:
    """Record `record()`'s device work into a graph; nothing has executed yet."""
    device.call("ttrl_capture_begin")
    device._capturing = True
    try:
        result = record()
        handle = C.c_void_p()
        device._capturing = False
        device.call("ttrl_capture_end", C.byref(handle))
    except BaseException as e:
        device._capturing = False
        _lib.lib().ttrl_capture_abort(device.ctx)
        if isinstance(e, (KeyboardInterrupt, SystemExit)):
            raise
        if HOST_READ_DURING_CAPTURE in str(e) or "not allowed while a graph is being captured" in str(e):
            raise TraceCaptureError(
                "graph capture failed because the captured work reads a tensor back to host or writes "
                "one from host (.numpy(), to_host(...), restore_in_place), which a captured graph cannot "
                "contain. Move every host transfer outside the capture. Device error: " + str(e)
            ) from e
        raise TraceCaptureError(f"graph capture failed: {e}") from e
    return CapturedTrace(device, handle), result
