"""Events that order work across HIP graphs, eager launches and streams.

The reference orders its writers and their consumers with external CUDA
events (``torch.cuda.Event(external=True)``, recorded and waited on inside
graph captures: kernels/pool.py:131-135, 338-355; kernels/writeback.py:43,
103, 110-116).  PyTorch-ROCm refuses external events, and HIP refuses
``hipEventRecordExternal`` under capture, but a capture accepts explicit
event nodes.  ``GraphEvent`` wraps a HIP event owned by the library
(``sq_event_*`` in include/stepquant_hip.h): ``record``/``wait`` act on the
stream at once, or, while the stream is capturing, add an event record /
wait node to the graph being captured.  A record node re-records the event
on every replay; a wait node makes the work captured after it wait for the
event's latest record, made by eager work or by another graph.
"""
from __future__ import annotations

import ctypes

from .. import _native as N


class GraphEvent:
    """A HIP event usable across graphs (created on first use)."""

    def __init__(self):
        self._handle = None

    @property
    def handle(self):
        if self._handle is None:
            h = ctypes.c_void_p()
            N.check(N.lib().sq_event_create(ctypes.byref(h)), "event create")
            self._handle = h
        return self._handle

    def record(self, stream=None):
        N.check(N.lib().sq_event_record(self.handle, N.stream_handle(stream)), "event record")

    def wait(self, stream=None):
        N.check(N.lib().sq_event_wait(N.stream_handle(stream), self.handle), "event wait")

    def query(self) -> bool:
        rc = N.lib().sq_event_query(self.handle)
        if rc not in (0, 1):
            N.check(rc, "event query")
        return rc == 0

    def synchronize(self):
        N.check(N.lib().sq_event_synchronize(self.handle), "event synchronize")

    def __del__(self):
        handle, self._handle = self._handle, None
        if handle is not None and N is not None and N._lib is not None:
            N._lib.sq_event_destroy(handle)


def wait_for(stream, event):
    """Order ``stream`` after ``event`` (a torch event or a GraphEvent)."""
    if isinstance(event, GraphEvent):
        event.wait(stream)
    else:
        stream.wait_event(event)


def capture_id(stream):
    """Identifier of the capture ``stream`` takes part in, or None."""
    capturing, ident = ctypes.c_int32(), ctypes.c_uint64()
    N.check(N.lib().sq_stream_capture_id(N.stream_handle(stream), ctypes.byref(capturing),
                                         ctypes.byref(ident)), "capture id")
    return ident.value if capturing.value == 1 else None
