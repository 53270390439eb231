"""HIP graph capture of fixed-buffer launch plans.

Same contract as the reference's CudaGraph (src/tensor/providers/cuda/graph.py:8-98):
capture submits only already-loaded kernels on the session stream; allocation,
copies and host reads happen outside the callback; buffer contents may change
between replays; a replay is refused once a retained resource was released.
"""

from __future__ import annotations

import ctypes as c

from tensor_amd import _native
from tensor_amd._native import HipError


class HipGraph:
    def __init__(self, device, submit, *, resources=()):
        device._check()
        self.device = device
        self.resources = tuple(resources)
        self.executable = 0
        self._closed = False
        self._generation = device._generation
        _native.call("tensor_hip_capture_begin", device.stream)
        try:
            submit()
        except BaseException:
            handle = c.c_uint64()
            try:
                _native.call("tensor_hip_capture_end", device.stream, c.byref(handle))
            except HipError:
                pass
            if handle.value:
                _native.call("tensor_hip_graph_destroy", handle.value)
            self._closed = True
            raise
        handle = c.c_uint64()
        try:
            _native.call("tensor_hip_capture_end", device.stream, c.byref(handle))
        except BaseException:
            self._closed = True
            raise
        self.executable = handle.value
        device._graphs.add(self)

    def launch(self):
        self.device._check()
        if self._closed or self._generation != self.device._generation:
            raise HipError("HipGraph", 3, "HIP graph is released or belongs to an old session")
        for resource in self.resources:
            while resource is not None:
                if getattr(resource, "_released", False) or getattr(resource, "_generation", self._generation) != self._generation:
                    raise HipError("HipGraph", 3, "HIP graph references a released resource")
                resource = getattr(resource, "_base", None)
        _native.call("tensor_hip_graph_launch", self.executable, self.device.stream)

    replay = launch

    def _dispose(self):
        if not self._closed:
            self._closed = True
            self.device._graphs.discard(self)
            _native.call("tensor_hip_graph_destroy", self.executable)

    def close(self):
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
