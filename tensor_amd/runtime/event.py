"""Completion events on a session's stream: the reference's Event surface
(src/tensor/runtime/event.py: ``descriptor``, ``release``, the provider/device check and its
error), plus ``synchronize``.

An event marks the work enqueued before it; the buffers that work uses stay borrowed until the
host waits on it or the device is synchronized.  In this build the session's ``Registry`` owns
its events by ticket: an event is valid while the registry that issued it is still its device's
current one (a reopened session has a new registry) and still lists it, so releasing an event or
closing its session invalidates it and its descriptor in one place, and a descriptor resolves to
its event by a dictionary lookup.
"""

from __future__ import annotations

import ctypes as c

from tensor_amd.runtime.abi import ABI_MAJOR, EventDescriptor
from tensor_amd.runtime.errors import TensorRuntimeError

TENSOR_EVENT_KNOWN_COMPLETE = 1  # set by providers whose launches complete before they return


class Event:
    def __init__(self, device, handle):
        self.device, self.handle = device, handle
        registry = device._registry
        self._registry, self._ticket = registry, registry.ticket()
        flags = 0 if "async_launch" in device.capabilities else TENSOR_EVENT_KNOWN_COMPLETE
        self._descriptor = EventDescriptor(ABI_MAJOR, c.sizeof(EventDescriptor), device.device_type, device.ordinal,
                                           device._session_id, self._ticket, flags, 0)
        registry.events[self._ticket] = self

    @property
    def _released(self) -> bool:
        return self._registry.events.get(self._ticket) is not self

    def _issued_for(self, device) -> bool:
        mine = self.device
        return (mine._registry is self._registry and not self._released
                and (device.device_type, device.ordinal) == (mine.device_type, mine.ordinal))

    @property
    def descriptor(self):
        """A copy of the native descriptor that names this event inside its session."""
        self._check(self.device)
        return EventDescriptor.from_buffer_copy(self._descriptor)

    def _check(self, device) -> None:
        if not self._issued_for(device):
            raise TensorRuntimeError("event is released or belongs to a different provider/device")
        self.device._check()

    def synchronize(self) -> None:
        """Block the host until the work recorded before this event has finished."""
        self._check(self.device)
        self.device._synchronize_event(self)

    def release(self) -> None:
        if self._released:
            return
        self._check(self.device)
        self.device._dispose_event(self)
        del self._registry.events[self._ticket]
