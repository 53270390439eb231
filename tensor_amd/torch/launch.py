"""Bind the Tensor call ABI once per shape, rebind pointers per call, and submit on
PyTorch's current stream.

Behaviour of packages/tensor-torch/src/tensor_torch/runtime/launch.py:101-226
and runtime/prepared.py:11-60.  The first call for a given set of shapes,
dtypes and scalar values imports every tensor by kDLROCM DLPack — the
provider checks that each pointer is device memory of the session's device —
and keeps the validated ``TensorCallV1`` descriptors in a per-kernel cache (64
entries, least recently used dropped).  Later calls write the tensors' data
pointers and the stream into those descriptors and call the entry point: no
import, no allocation, no synchronisation.  ctypes releases the GIL around the
native call, which is what the reference's submission shim
(native/launch.c:19-40) is for.
"""

from __future__ import annotations

import ctypes as c
import importlib
import os
import threading
from contextlib import nullcontext

import torch

from tensor_amd.runtime.abi import DEVICE_ROCM, CallDescriptor, StreamDescriptor
from tensor_amd.runtime.signature import SCALAR_TYPES, buffer_argument, scalar_value
from tensor_amd.torch.session import current_stream, session

PREPARED_CACHE = 64

# The C++ executor (executor.cpp) is built against torch's non-stable ABI: only a module
# built for this torch's major/minor version is imported.  TENSOR_AMD_TORCH_NATIVE=0
# keeps every launch on the Python path.
_executor = None
if os.environ.get("TENSOR_AMD_TORCH_NATIVE", "1") != "0":
    _major, _minor = torch.__version__.split("+")[0].split(".")[:2]
    try:
        _executor = importlib.import_module(f"tensor_amd.torch._executor_{_major}_{_minor}")
    except ImportError:
        pass


def native_executor():
    """The native executor module in use, or None."""
    return _executor


class _Call:
    """Descriptor storage of one bound call (what the provider's ``_launch`` reads)."""

    def __init__(self, arguments, descriptor, retained):
        self.arguments, self.descriptor, self.retained = arguments, descriptor, retained

    @classmethod
    def of(cls, bound):
        return cls(bound.arguments, bound.descriptor, bound.storage)

    def copy(self):
        """Independent descriptors over the same shape/stride arrays."""
        arguments = type(self.arguments).from_buffer_copy(self.arguments)
        descriptor = CallDescriptor.from_buffer_copy(self.descriptor)
        descriptor.arguments = c.cast(arguments, c.POINTER(arguments._type_))
        return _Call(arguments, descriptor, self.retained)


def _slots(manifest):
    """(argument index, descriptor, alignment) of each ABI argument."""
    alignments = {d["name"]: d.get("alignment", 256) for d in manifest["arguments"] if buffer_argument(d)}
    return [(index, d, alignments.get(d["name"], 1))
            for index, d in enumerate(manifest.get("abi", manifest["arguments"]))]


def native_plan(kernel, executable, call, args, outputs, *, fixed):
    """A native executor Plan over ``call``'s descriptors, or None without the executor.
    ``args`` are the kernel's inputs in order; tensors are bound by position."""
    if _executor is None:
        return None
    from tensor_amd import _native

    tensors = [v for d, v in zip(kernel.inputs, args) if buffer_argument(d)]
    positions = {d["name"]: i for i, d in enumerate(d for d in kernel.inputs if buffer_argument(d))}
    positions.update((d["name"], len(tensors) + i) for i, d in enumerate(kernel.outputs))
    bindings = [(index, positions[d["name"]], alignment) for index, d, alignment in kernel._slots
                if buffer_argument(d)]
    if executable.manifest.get("kind") == "hsaco":
        entry = c.cast(_native.library().tensor_hip_module_launch_v1, c.c_void_p).value
        function = executable.function
    else:
        entry, function = c.cast(executable.function, c.c_void_p).value, 0
    return _executor.Plan(executable.manifest["entrypoint"], entry, function, c.addressof(call.descriptor),
                          tuple(tensors), tuple(outputs), bindings, fixed)


def _bind(device, executable, manifest, values, stream):
    """Validate one call through DLPack imports; returns descriptors that outlive the imports."""
    borrowed, ordered = [], []
    constants = manifest.get("constants", {})
    try:
        for descriptor in manifest["arguments"]:
            name = descriptor["name"]
            if name in constants:
                continue
            value = values[name]
            if buffer_argument(descriptor):
                buffer = device.from_dlpack(value.detach(), stream=stream.cuda_stream)
                borrowed.append(buffer)
                ordered.append(buffer)
            else:
                ordered.append(value)
        return _Call.of(executable.bind(*ordered))
    finally:
        # The descriptors keep the buffers' shape arrays; the DLPack owners go back now.
        for buffer in borrowed:
            buffer._dispose()


def _rebind(call, slots, values, stream, ordinal):
    for index, descriptor, alignment in slots:
        name = descriptor["name"]
        argument = call.arguments[index]
        if buffer_argument(descriptor):
            value = values[name]
            pointer = value.data_ptr()
            if pointer % alignment:
                raise ValueError(f"{name} has insufficient pointer alignment")
            value.record_stream(stream)
            argument.buffer.address = pointer
        elif name in values:
            scalar = SCALAR_TYPES[descriptor["dtype"]](scalar_value(values[name], descriptor["dtype"], name))
            c.memmove(c.addressof(argument) + type(argument).scalar.offset, c.byref(scalar), c.sizeof(scalar))
    call.descriptor.stream = StreamDescriptor(DEVICE_ROCM, ordinal, stream.cuda_stream)


def _key(kernel, ordinal, values):
    symbols = kernel.manifest.get("symbols", {})
    parts = []
    for descriptor in kernel.manifest["arguments"]:
        name = descriptor["name"]
        if name not in values:
            continue
        value = values[name]
        if buffer_argument(descriptor):
            parts.append((name, tuple(value.shape), value.dtype))
        else:
            parts.append((name, type(value), value if name in symbols else None))
    return ordinal, tuple(parts)


def launch(kernel, args, outputs, *, contract=None, trusted_outputs=False, enqueue=True):
    """Launch ``kernel`` on its inputs and caller-owned outputs, on the current stream."""
    expected, placement = contract or kernel.metadata(args)
    if len(outputs) != len(expected):
        raise ValueError("wrong output count")
    tensors = [v for d, v in zip(kernel.inputs, args) if buffer_argument(d)]
    for position, (out, (shape, dtype)) in enumerate(zip(outputs, expected)):
        if (not isinstance(out, torch.Tensor) or tuple(out.shape) != tuple(shape) or out.dtype != dtype
                or out.device != placement or not out.is_contiguous()):
            raise ValueError("output shape, dtype, layout or device mismatch")
        if not trusted_outputs and any(out.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()
                                       for v in tensors + list(outputs[:position])):
            raise ValueError("outputs must not alias inputs or each other")
    ordinal = placement.index if placement.index is not None else torch.cuda.current_device()
    with kernel._lock, torch.cuda.device(ordinal):
        device = session(ordinal)
        executable = kernel._executable(device, ordinal)
        stream = current_stream(ordinal)
        values = dict(zip((d["name"] for d in kernel.inputs), args))
        values.update(zip((d["name"] for d in kernel.outputs), outputs))
        key = _key(kernel, ordinal, values)
        call = kernel._prepared.get(key)
        if call is None:
            call = kernel._prepared[key] = _bind(device, executable, kernel.manifest, values, stream)
            if len(kernel._prepared) > PREPARED_CACHE:
                kernel._prepared.popitem(last=False)
        kernel._prepared.move_to_end(key)
        _rebind(call, kernel._slots, values, stream, ordinal)
        if enqueue:
            device._launch(executable, call)
        return executable, call, tuple(tensors) + tuple(outputs), stream


class Prepared:
    """A call over fixed tensors, submitted again on each ``()`` on the current stream.

    Changing the tensors' data in place is supported; changing their storage,
    shape, strides, dtype or device is refused.
    """

    def __init__(self, kernel, state, args, outputs):
        self.executable, call, self.tensors, stream = state
        self.call = call.copy()  # later launches of the kernel rewrite the cached descriptors
        self.args, self.outputs = args, outputs
        self.device = self.executable.device
        self.ordinal = self.device.ordinal
        self.metadata = [(tuple(t.shape), tuple(t.stride()), t.dtype, t.device, t.data_ptr()) for t in self.tensors]
        self.streams = {stream.cuda_stream: stream}
        self.lock = threading.RLock()
        self._native = native_plan(kernel, self.executable, self.call, args, outputs, fixed=True)

    def __call__(self):
        if not self.device._open or self.executable._released:
            raise RuntimeError("prepared call belongs to a closed session")
        if self._native is not None:
            self._native()
            return
        for tensor, (shape, stride, dtype, device, pointer) in zip(self.tensors, self.metadata):
            if (tensor.data_ptr() != pointer or tuple(tensor.shape) != shape or tuple(tensor.stride()) != stride
                    or tensor.dtype != dtype or tensor.device != device):
                raise ValueError("prepared tensor metadata or storage changed")
        guard = torch.cuda.device(self.ordinal) if torch.cuda.current_device() != self.ordinal else nullcontext()
        with self.lock, guard:
            stream = current_stream(self.ordinal)
            if stream.cuda_stream not in self.streams:
                for tensor in self.tensors:
                    tensor.record_stream(stream)
                self.streams[stream.cuda_stream] = stream
            self.call.descriptor.stream = StreamDescriptor(DEVICE_ROCM, self.ordinal, stream.cuda_stream)
            self.device._launch(self.executable, self.call)
