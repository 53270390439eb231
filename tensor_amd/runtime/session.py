"""Executable and event ownership within one device session.

Mirrors src/tensor/runtime/session.py:13-74: descriptors handed out by a
session resolve only inside that live session.
"""

from __future__ import annotations

import ctypes as c
from itertools import count

from tensor_amd.runtime.abi import ABI_MAJOR, EventDescriptor, ExecutableDescriptor

_identities = count(1)


class Session:
    """Common executable/event bookkeeping; providers own the device resources."""

    def _start_session(self):
        self._session_id = next(_identities)
        self._executables = {}

    def _resolve(self, descriptor, kind, expected_type):
        if (
            not isinstance(descriptor, expected_type)
            or descriptor.abi_version != ABI_MAJOR
            or descriptor.struct_size < c.sizeof(expected_type)
        ):
            raise self.error(f"unsupported {kind} descriptor ABI")
        self._check()
        if (
            descriptor.device_type != self.device_type
            or descriptor.device_ordinal != self.ordinal
            or descriptor.session != self._session_id
        ):
            raise self.error(f"{kind} descriptor belongs to a different device session")

    def get_executable(self, descriptor):
        self._resolve(descriptor, "executable", ExecutableDescriptor)
        executable = self._executables.get(descriptor.handle)
        if executable is None:
            raise self.error("executable handle is released or unknown")
        expected = executable._descriptor
        if (
            descriptor.argument_count != expected.argument_count
            or descriptor.flags != expected.flags
            or bytes(descriptor.workspace) != bytes(expected.workspace)
        ):
            raise self.error("executable descriptor metadata mismatch")
        return executable

    def get_event(self, descriptor):
        self._resolve(descriptor, "event", EventDescriptor)
        for event in self._events:
            if event._descriptor.handle == descriptor.handle:
                if descriptor.flags != event._descriptor.flags or descriptor.reserved:
                    raise self.error("event descriptor metadata mismatch")
                return event
        raise self.error("event handle is released or unknown")
