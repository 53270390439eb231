"""HIP graphs of already-bound launches.

The contract is that of the reference's CudaGraph (src/tensor/providers/cuda/graph.py): capture
enqueues only loaded kernels on the session stream; allocations, copies and host reads happen
outside the capture; buffer contents may change between replays; a graph whose resources were
released is never replayed.

How this build does it: a ``_Capture`` context owns one capture of the session stream, so the
capture is ended on every path out of the callback and the provider's capture log is always
detached.  While it is open, every launch the provider submits adds the buffers its call retains
to the log, so a graph knows the device memory its kernels touch without being told (callers may
add more with ``resources``).  A replay first checks that each of them is live in the graph's
session, because a kernel node replayed over freed memory would read or write whatever owns that
memory now; buffers and their views share one storage record, so one test per buffer covers
every view of it.
"""

from __future__ import annotations

import ctypes as c

from tensor_amd import _native
from tensor_amd._native import HipError


class _Capture:
    """One open capture of a session's stream.  ``handle`` is the executable graph once the
    block completed; a block that raised leaves no graph behind."""

    def __init__(self, device):
        self.device, self.recorded, self.handle = device, [], 0

    def __enter__(self):
        self.device._capture_log = self.recorded
        _native.call("tensor_hip_capture_begin", self.device.stream)
        return self

    def __exit__(self, kind, error, trace):
        self.device._capture_log = None
        graph = c.c_uint64()
        try:
            _native.call("tensor_hip_capture_end", self.device.stream, c.byref(graph))
        except HipError:
            if kind is None:
                raise
            # the callback's error is the one to report; its capture may have been invalidated
        if kind is None:
            self.handle = graph.value
        elif graph.value:
            _native.call("tensor_hip_graph_destroy", graph.value)
        return False


def _stale(resource, generation) -> bool:
    return bool(getattr(resource, "_released", False)) or getattr(resource, "_generation", generation) != generation


class HipGraph:
    def __init__(self, device, submit, *, resources=()):
        device._check()
        self.device, self._generation = device, device._generation
        self._closed, self.handle = True, 0
        with _Capture(device) as capture:
            submit()
        self.handle, self._closed = capture.handle, False
        self.resources = tuple({id(r): r for r in (*resources, *capture.recorded)}.values())
        device._graphs.add(self)

    def replay(self) -> None:
        """Launch the captured work again on the session stream."""
        device = self.device
        device._check()
        if self._closed or self._generation != device._generation:
            raise HipError("HipGraph", 3, "HIP graph is released or belongs to an old session")
        if any(_stale(resource, self._generation) for resource in self.resources):
            raise HipError("HipGraph", 3, "HIP graph references a released resource")
        _native.call("tensor_hip_graph_launch", self.handle, device.stream)

    launch = replay

    def _dispose(self) -> None:
        if self._closed:
            return
        self._closed = True
        self.device._graphs.discard(self)
        _native.call("tensor_hip_graph_destroy", self.handle)

    def close(self) -> None:
        """Wait for the stream, then destroy the graph and drop its resources."""
        if self._closed:
            return
        self.device._check()
        self.device.synchronize()
        self._dispose()
        self.resources = ()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
