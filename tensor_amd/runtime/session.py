"""Native descriptors handed out by a device session, and their resolution.

Executables and events can be named across the C boundary by descriptors
(TensorExecutableV1, TensorEventV1) that carry the device, a session id and a handle.  A
descriptor resolves only in the live session that issued it, and only while its object is
alive and its metadata is unchanged -- the reference's rule (src/tensor/runtime/session.py,
docs/reference/runtime-abi.md:127-142).  Each session keeps a ``Registry`` of what it issued.
"""

from __future__ import annotations

import ctypes as c
import itertools

from tensor_amd.runtime.abi import ABI_MAJOR, EventDescriptor, ExecutableDescriptor

_sessions = itertools.count(1)


class Registry:
    """What one session issued, by ticket: executables and events."""

    def __init__(self):
        self.session_id = next(_sessions)
        self.executables = {}
        self.events = {}
        self._tickets = itertools.count(1)

    def ticket(self) -> int:
        return next(self._tickets)


class Session:
    """Descriptor bookkeeping shared by providers: ``_start_session`` when a session opens,
    ``get_executable`` / ``get_event`` to resolve descriptors from native code."""

    def _start_session(self) -> None:
        self._registry = Registry()

    @property
    def _session_id(self) -> int:
        return self._registry.session_id

    @property
    def _executables(self) -> dict:
        return self._registry.executables

    @property
    def _events(self) -> list:
        """The live events of the current (or last) session."""
        registry = getattr(self, "_registry", None)
        return list(registry.events.values()) if registry is not None else []

    def _owns(self, descriptor, expected_type, kind: str) -> None:
        if type(descriptor) is not expected_type or descriptor.abi_version != ABI_MAJOR \
                or descriptor.struct_size < c.sizeof(expected_type):
            raise self.error(f"unsupported {kind} descriptor ABI")
        self._check()
        origin = (descriptor.device_type, descriptor.device_ordinal, descriptor.session)
        if origin != (self.device_type, self.ordinal, self._session_id):
            raise self.error(f"{kind} descriptor belongs to a different device session")

    def get_executable(self, descriptor):
        self._owns(descriptor, ExecutableDescriptor, "executable")
        executable = self._executables.get(descriptor.handle)
        if executable is None:
            raise self.error("executable handle is released or unknown")
        issued = executable._descriptor
        same = (descriptor.argument_count == issued.argument_count and descriptor.flags == issued.flags
                and bytes(descriptor.workspace) == bytes(issued.workspace))
        if not same:
            raise self.error("executable descriptor metadata mismatch")
        return executable

    def get_event(self, descriptor):
        self._owns(descriptor, EventDescriptor, "event")
        match = self._registry.events.get(descriptor.handle)
        if match is None:
            raise self.error("event handle is released or unknown")
        if descriptor.flags != match._descriptor.flags or descriptor.reserved:
            raise self.error("event descriptor metadata mismatch")
        return match
