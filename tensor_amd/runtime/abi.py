"""ctypes mirror of the C call ABI (include/tensor/abi.h) and the bound call.

The structure layouts and ids are the reference's descriptors, byte for byte
(src/tensor/runtime/abi.py:16-133, src/tensor/include/tensor/abi.h:37-131): they are
the interface a provider consumes.  ``BoundCall`` holds the TensorCallV1 storage of one
validated call, which a provider borrows for each submission.
"""

from __future__ import annotations

import ctypes as c
import sys

from tensor_amd.runtime.signature import SCALAR_TYPES, scalar_value

ABI_MAJOR = 1
ABI_MINOR = 3
DEVICE_CPU = 1
DEVICE_ROCM = 10
DTYPE_NAMES = (
    "bool", "int8", "uint8", "int16", "uint16", "int32", "uint32",
    "int64", "uint64", "float16", "float32", "float64", "bfloat16",
)
DTYPES = {name: index for index, name in enumerate(DTYPE_NAMES, 1)}
CAPABILITIES = frozenset(
    {"contiguous", "scalars", "symbolic_shapes", "executable_descriptors", "no_external_workspace"}
)
KNOWN_CAPABILITIES = CAPABILITIES | {"opaque_buffer_handles", "bfloat16_storage", "cuda_tensor_maps"}


class BufferDescriptor(c.Structure):
    _fields_ = [
        ("address", c.c_uint64),
        ("byte_size", c.c_uint64),
        ("shape", c.POINTER(c.c_int64)),
        ("strides", c.POINTER(c.c_int64)),
        ("rank", c.c_uint32),
        ("dtype", c.c_uint32),
        ("device_type", c.c_uint32),
        ("device_ordinal", c.c_int32),
    ]


class Argument(c.Structure):
    _fields_ = [
        ("kind", c.c_uint32),
        ("dtype", c.c_uint32),
        ("buffer", BufferDescriptor),
        ("scalar", c.c_uint64),
    ]


class StreamDescriptor(c.Structure):
    _fields_ = [("device_type", c.c_uint32), ("device_ordinal", c.c_int32), ("handle", c.c_uint64)]


class CallDescriptor(c.Structure):
    _fields_ = [
        ("abi_version", c.c_uint32),
        ("struct_size", c.c_uint32),
        ("arguments", c.POINTER(Argument)),
        ("argument_count", c.c_uint32),
        ("flags", c.c_uint32),
        ("grid", c.c_uint32 * 3),
        ("block", c.c_uint32 * 3),
        ("shared_memory_bytes", c.c_uint64),
        ("stream", StreamDescriptor),
    ]


class ErrorDescriptor(c.Structure):
    _fields_ = [("code", c.c_int32), ("message", c.c_char * 508)]


class WorkspaceRequirements(c.Structure):
    _fields_ = [
        ("byte_size", c.c_uint64),
        ("alignment", c.c_uint32),
        ("device_type", c.c_uint32),
        ("flags", c.c_uint32),
        ("reserved", c.c_uint32),
    ]


class ExecutableDescriptor(c.Structure):
    _fields_ = [
        ("abi_version", c.c_uint32),
        ("struct_size", c.c_uint32),
        ("device_type", c.c_uint32),
        ("device_ordinal", c.c_int32),
        ("session", c.c_uint64),
        ("handle", c.c_uint64),
        ("argument_count", c.c_uint32),
        ("flags", c.c_uint32),
        ("workspace", WorkspaceRequirements),
    ]


class EventDescriptor(c.Structure):
    _fields_ = [
        ("abi_version", c.c_uint32),
        ("struct_size", c.c_uint32),
        ("device_type", c.c_uint32),
        ("device_ordinal", c.c_int32),
        ("session", c.c_uint64),
        ("handle", c.c_uint64),
        ("flags", c.c_uint32),
        ("reserved", c.c_uint32),
    ]


SIZES = {
    BufferDescriptor: 48, Argument: 64, StreamDescriptor: 16, CallDescriptor: 72,
    ErrorDescriptor: 512, WorkspaceRequirements: 24, ExecutableDescriptor: 64, EventDescriptor: 40,
}
for _structure, _size in SIZES.items():
    assert c.sizeof(_structure) == _size, (_structure.__name__, c.sizeof(_structure))


_HOST_OK = c.sizeof(c.c_void_p) == 8 and sys.byteorder == "little"


def check_requirement(requirement: dict, capabilities=KNOWN_CAPABILITIES) -> None:
    """Accept a manifest's ``runtime_abi`` only for ABI major 1, a minor this runtime knows and
    capabilities the provider has (the reference's rule, src/tensor/runtime/abi.py:164-193)."""
    if not isinstance(requirement, dict) or sorted(requirement) != ["major", "minor", "required_capabilities"]:
        raise ValueError("unsupported Tensor runtime ABI version")
    major, minor, needed = requirement["major"], requirement["minor"], requirement["required_capabilities"]
    if type(major) is not int or major != ABI_MAJOR or type(minor) is not int or not 0 <= minor <= ABI_MINOR:
        raise ValueError("unsupported Tensor runtime ABI version")
    if not isinstance(needed, list) or not all(isinstance(name, str) for name in needed) \
            or len(needed) != len(set(needed)):
        raise ValueError("invalid runtime capabilities")
    absent = sorted(set(needed).difference(capabilities))
    if absent:
        raise ValueError(f"missing runtime capabilities: {absent}")


def _scalar_bits(value, dtype: str) -> int:
    """The little-endian payload of a scalar argument: its value in the low bytes, zeros above."""
    raw = bytes(SCALAR_TYPES[dtype](value))
    return int.from_bytes(raw, "little")


class BoundCall:
    """A validated call, packed once into TensorCallV1 storage and submitted any number of times.

    ``values`` maps argument names to buffers and canonical scalars; a scalar the caller did not
    pass is a manifest constant (fixed when the executable was loaded, such as a GGUF kernel's
    GGML type) or a bound dimension of the same name.  The buffers are retained in ``storage``
    so their descriptors stay valid while the call lives.
    """

    def __init__(self, executable, values: dict, symbols: dict, launch: dict, stream: StreamDescriptor):
        if not _HOST_OK:
            raise ValueError("Tensor ABI 1 needs a 64-bit little-endian host")
        signature = executable.signature
        self.executable = executable
        self.storage = []
        self.arguments = (Argument * len(signature.abi))()
        for slot, (name, dtype, is_buffer) in zip(self.arguments, signature.abi):
            slot.dtype = DTYPES[dtype]
            if is_buffer:
                buffer = values[name]
                self.storage.append(buffer)
                slot.kind = 1
                slot.buffer = buffer._descriptor
            else:
                value = values[name] if name in values else signature.constants.get(name, symbols.get(name))
                if value is None:
                    raise ValueError(f"scalar {name} has no value")
                slot.kind = 2
                slot.scalar = _scalar_bits(scalar_value(value, dtype, name), dtype)
        grid, block = (c.c_uint32 * 3)(*launch["grid"]), (c.c_uint32 * 3)(*launch["block"])
        self.descriptor = CallDescriptor(ABI_MAJOR, c.sizeof(CallDescriptor), self.arguments, len(self.arguments),
                                         0, grid, block, launch["shared_memory_bytes"], stream)

    @property
    def buffers(self) -> tuple:
        return tuple(self.storage)

    def launch(self) -> None:
        """Submit again: the descriptors are reused as they are (no allocation, no re-binding);
        a released executable or buffer is refused before the provider sees the call.  The
        checks read Python state only; the provider's launch is the one native call (its device
        check costs none while the thread's device stays set)."""
        executable = self.executable
        fault = executable._fault()
        if fault:
            raise executable.device.error(fault)
        generation = executable._generation
        for buffer in self.storage:
            if buffer._released or buffer._generation != generation:
                buffer._check()  # raises the buffer's own error
        executable.device._launch(executable, self)

    __call__ = launch
