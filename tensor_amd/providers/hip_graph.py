"""HIP graphs of already-bound launches (the contract of the reference's CudaGraph,
src/tensor/providers/cuda/graph.py: capture enqueues only loaded kernels on the session
stream; allocations, copies and host reads happen outside the capture; buffer contents may
change between replays; a graph whose resources were released is never replayed).

Every launch the provider submits while a capture is open records the buffers its call
retains, so a graph knows the device memory its kernels touch without being told; callers
may add more with ``resources``.  Each replay checks that all of them are still live before
``hipGraphLaunch``, because a kernel node replayed over freed memory would read or write
whatever owns that memory now.
"""

from __future__ import annotations

import ctypes as c

from tensor_amd import _native
from tensor_amd._native import HipError


def _live(buffer, generation) -> bool:
    link = buffer
    while link is not None:
        if getattr(link, "_released", False) or getattr(link, "_generation", generation) != generation:
            return False
        link = getattr(link, "_base", None)
    return True


class HipGraph:
    def __init__(self, device, submit, *, resources=()):
        device._check()
        self.device = device
        self._generation = device._generation
        self._closed = False
        self.handle = 0
        recorded = []
        device._capture_log = recorded
        _native.call("tensor_hip_capture_begin", device.stream)
        handle = c.c_uint64()
        try:
            submit()
        except BaseException:
            device._capture_log = None
            try:
                _native.call("tensor_hip_capture_end", device.stream, c.byref(handle))
            except HipError:
                pass
            if handle.value:
                _native.call("tensor_hip_graph_destroy", handle.value)
            self._closed = True
            raise
        device._capture_log = None
        try:
            _native.call("tensor_hip_capture_end", device.stream, c.byref(handle))
        except BaseException:
            self._closed = True
            raise
        self.handle = handle.value
        unique = {id(b): b for b in [*resources, *recorded]}
        self.resources = tuple(unique.values())
        device._graphs.add(self)

    def replay(self) -> None:
        """Launch the captured work again on the session stream."""
        self.device._check()
        if self._closed or self._generation != self.device._generation:
            raise HipError("HipGraph", 3, "HIP graph is released or belongs to an old session")
        for buffer in self.resources:
            if not _live(buffer, self._generation):
                raise HipError("HipGraph", 3, "HIP graph references a released resource")
        _native.call("tensor_hip_graph_launch", self.handle, self.device.stream)

    launch = replay

    def _dispose(self) -> None:
        if not self._closed:
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
