"""Completion events on a session's stream (the reference's Event surface,
src/tensor/runtime/event.py).  An event marks the work enqueued before it; the buffers that
work uses stay borrowed until the host waits on it or the device is synchronized."""

from __future__ import annotations

import ctypes as c

from tensor_amd.runtime.abi import ABI_MAJOR, EventDescriptor
from tensor_amd.runtime.errors import TensorRuntimeError


class Event:
    def __init__(self, device, handle):
        self.device, self.handle = device, handle
        self._session = device._generation
        self._released = False
        ticket = device._registry.ticket()
        flags = 0 if "async_launch" in device.capabilities else 1  # TENSOR_EVENT_KNOWN_COMPLETE
        self._descriptor = EventDescriptor(ABI_MAJOR, c.sizeof(EventDescriptor), device.device_type, device.ordinal,
                                           device._session_id, ticket, flags, 0)

    @property
    def descriptor(self):
        """A copy of the native descriptor that names this event inside its session."""
        self._check(self.device)
        return EventDescriptor.from_buffer_copy(self._descriptor)

    def _check(self, device) -> None:
        mine = self.device
        if self._released or self._session != mine._generation \
                or (device.device_type, device.ordinal) != (mine.device_type, mine.ordinal):
            raise TensorRuntimeError("event is released or belongs to a different provider/device")
        mine._check()

    def synchronize(self) -> None:
        """Block the host until the work recorded before this event has finished."""
        self._check(self.device)
        self.device._synchronize_event(self)

    def release(self) -> None:
        if self._released:
            return
        self._check(self.device)
        self.device._dispose_event(self)
        self.device._events.discard(self)
        self._released = True
