"""ctypes mirror of the C call ABI (include/tensor/abi.h) and the call builder.

Layouts and ids are those of the reference's descriptors
(src/tensor/runtime/abi.py:16-133, src/tensor/include/tensor/abi.h:37-131);
``BoundCall`` owns the descriptor storage a provider borrows for one submission
(src/tensor/runtime/abi.py:196-261).
"""

from __future__ import annotations

import ctypes as c
import sys

from tensor_amd.runtime.signature import SCALAR_TYPES, buffer_argument, evaluate, scalar_value

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


def check_requirement(requirement: dict, capabilities=KNOWN_CAPABILITIES) -> None:
    """Reject unknown major versions, newer minors and missing capabilities
    (reference: src/tensor/runtime/abi.py:164-193)."""
    if (
        not isinstance(requirement, dict)
        or set(requirement) != {"major", "minor", "required_capabilities"}
        or type(requirement["major"]) is not int
        or requirement["major"] != ABI_MAJOR
        or type(requirement["minor"]) is not int
        or not 0 <= requirement["minor"] <= ABI_MINOR
    ):
        raise ValueError("unsupported Tensor runtime ABI version")
    required = requirement["required_capabilities"]
    if not isinstance(required, list) or any(not isinstance(n, str) for n in required) or len(set(required)) != len(required):
        raise ValueError("invalid runtime capabilities")
    missing = set(required) - set(capabilities)
    if missing:
        raise ValueError(f"missing runtime capabilities: {sorted(missing)}")


class BoundCall:
    """Descriptor storage for one validated call, kept alive while borrowed.

    Scalar arguments come from the supplied values, the manifest's
    ``constants`` (values an executable fixes when it is loaded, such as the
    GGML type of a GGUF kernel) or the bound dimension symbols.
    """

    def __init__(self, device, manifest, values, symbols, launch, *, validated=False, executable=None):
        if c.sizeof(c.c_void_p) != 8 or sys.byteorder != "little":
            raise ValueError("Tensor ABI 1 requires a 64-bit little-endian host")
        abi = manifest.get("abi", [dict(item, kind="buffer") for item in manifest["arguments"]])
        constants = manifest.get("constants", {})
        self.storage = []
        self.executable = executable
        self.arguments = (Argument * len(abi))()
        for argument, descriptor in zip(self.arguments, abi):
            name, dtype = descriptor["name"], descriptor["dtype"]
            argument.dtype = DTYPES[dtype]
            if buffer_argument(descriptor):
                value = values[name]
                self.storage.append(value)
                argument.kind = 1
                argument.buffer = value._descriptor
                continue
            if name in values:
                value = values[name]
            elif name in constants:
                value = constants[name]
            else:
                value = evaluate({"var": name}, symbols)
            scalar = SCALAR_TYPES[dtype](value if validated and name in values else scalar_value(value, dtype, name))
            argument.kind = 2
            c.memmove(c.addressof(argument) + Argument.scalar.offset, c.byref(scalar), c.sizeof(scalar))
        self.descriptor = CallDescriptor(
            ABI_MAJOR,
            c.sizeof(CallDescriptor),
            self.arguments,
            len(abi),
            0,
            (c.c_uint32 * 3)(*launch["grid"]),
            (c.c_uint32 * 3)(*launch["block"]),
            launch["shared_memory_bytes"],
            device.stream_descriptor(),
        )

    def launch(self):
        """Submit again with the retained descriptors (no allocation, no re-binding)."""
        if self.executable is None:
            raise ValueError("bind this call through Executable.bind before submission")
        self.executable._check()
        for buffer in self.storage:
            buffer._check()
        self.executable.device._launch(self.executable, self)

    __call__ = launch
