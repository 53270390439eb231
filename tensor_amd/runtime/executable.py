"""Loaded executables (the reference's Executable surface, src/tensor/runtime/executable.py):
``launch``, ``bind`` (a retained ``BoundCall``), ``prepare`` (allocate the declared outputs)
and ``__call__`` (allocate, launch, return the outputs).

Each executable compiles its manifest into a ``Signature`` once; a call is matched against
it by name and position, every buffer is checked to be live, on this device and aligned,
the symbols are derived from the buffers' shapes, and the launch geometry is checked against
the device's limits before anything is submitted.
"""

from __future__ import annotations

import ctypes as c
import math

from tensor_amd.runtime.abi import ABI_MAJOR, BoundCall, ExecutableDescriptor, WorkspaceRequirements
from tensor_amd.runtime.buffer import Buffer
from tensor_amd.runtime.signature import Signature


class Executable:
    def __init__(self, device, manifest: dict, module, function, image):
        self.device, self.manifest = device, manifest
        self.module, self.function, self._image = module, function, image
        self.signature = Signature(manifest)
        self._generation = device._generation
        self._released = False
        self._handle = device._registry.ticket()
        no_workspace = WorkspaceRequirements(0, 1, device.device_type, 0, 0)
        flags = 1 if "async_launch" in device.capabilities else 0  # TENSOR_EXEC_ASYNC
        self._descriptor = ExecutableDescriptor(ABI_MAJOR, c.sizeof(ExecutableDescriptor), device.device_type,
                                                device.ordinal, device._session_id, self._handle,
                                                len(self.signature.abi), flags, no_workspace)
        device._executables[self._handle] = self

    def __repr__(self):
        return f"Executable({self.manifest.get('name', self.manifest.get('entrypoint'))})"

    # -- lifetime -------------------------------------------------------------
    def _check(self) -> None:
        device = self.device
        if not device._open:
            raise device.error("device session is closed")
        if self._generation != device._generation:
            raise device.error("executable belongs to a previous device session")
        if self._released:
            raise device.error("executable has been released")

    @property
    def descriptor(self):
        self._check()
        return ExecutableDescriptor.from_buffer_copy(self._descriptor)

    def workspace_requirements(self):
        self._check()
        return WorkspaceRequirements.from_buffer_copy(self._descriptor.workspace)

    def release(self) -> None:
        if not self._released:
            self._check()
            self.device.synchronize()
            self._dispose()

    def _dispose(self) -> None:
        if self._released:
            return
        self.device._unload_executable(self)
        self._released = True
        self.device._executables.pop(self._handle, None)
        self.module = self.function = self._image = None

    def __enter__(self):
        self._check()
        return self

    def __exit__(self, *exc):
        self.release()

    # -- calls ----------------------------------------------------------------
    def _match(self, arguments: tuple, keywords: dict, *, outputs: bool):
        """Name every supplied value after its slot; keywords may also set dimension symbols."""
        slots = self.signature.parameters(outputs=outputs)
        if len(arguments) > len(slots):
            raise ValueError(f"kernel expects at most {len(slots)} arguments, received {len(arguments)}")
        values = {slot.name: value for slot, value in zip(slots, arguments)}
        names = {slot.name for slot in slots}
        dimensions = {}
        for name, value in keywords.items():
            if name in values:
                raise ValueError(f"argument {name} supplied twice")
            if name in names:
                values[name] = value
            elif name in self.signature.symbol_types:
                dimensions[name] = value
            else:
                raise ValueError(f"unknown kernel argument {name}")
        absent = sorted(names - values.keys())
        if absent:
            raise ValueError(f"missing kernel arguments: {absent}")
        for slot in slots:
            if slot.buffer:
                self._admit(slot, values[slot.name])
        return values, dimensions

    def _admit(self, slot, buffer) -> None:
        if not isinstance(buffer, Buffer):
            raise TypeError(f"{slot.name} must be a Tensor Buffer")
        if buffer.device is not self.device:
            raise ValueError(f"{slot.name} belongs to a different device session")
        link = buffer
        while link is not None:
            if link._released or link._generation != self._generation:
                raise self.device.error("buffer has been released")
            link = link._base
        if buffer.pointer % slot.alignment:
            raise ValueError(f"{slot.name} needs {slot.alignment}-byte pointer alignment")

    def _geometry(self, symbols: dict) -> dict:
        launch = self.signature.launch(symbols)
        limits = self.device.limits
        for field in ("grid", "block"):
            if any(v > limit for v, limit in zip(launch[field], limits[field])):
                raise ValueError(f"launch {field} exceeds this device's limits")
        if limits.get("threads") is not None and math.prod(launch["block"]) > limits["threads"]:
            raise ValueError("launch thread count exceeds this device's limit")
        return launch

    def bind(self, *arguments, **bindings) -> BoundCall:
        """Validate once and return a BoundCall for repeated, allocation-free submission.
        Bind again when shapes, scalars or storage change."""
        self._check()
        values, dimensions = self._match(arguments, bindings, outputs=True)
        symbols, values = self.signature.bind(values, dimensions)
        return BoundCall(self, values, symbols, self._geometry(symbols), self.device.stream_descriptor())

    def launch(self, *arguments, **bindings) -> None:
        """Launch with every buffer argument, outputs included."""
        self.device._launch(self, self.bind(*arguments, **bindings))

    def prepare(self, *inputs, **bindings):
        """Allocate the declared outputs for these inputs without launching; returns the full
        argument tuple, the dimensions the inputs did not fix, and the new outputs by name."""
        self._check()
        outputs = self.signature.outputs
        if not outputs:
            raise ValueError("artifact has no declared outputs; call launch with every buffer")
        values, dimensions = self._match(inputs, bindings, outputs=False)
        symbols, values = self.signature.bind(values, dimensions)
        created = {}
        try:
            for name in outputs:
                slot = self.signature.by_name[name]
                created[name] = self.device.empty(slot.shape(symbols), slot.dtype)
        except BaseException:
            for buffer in created.values():
                buffer.release()
            raise
        values.update(created)
        ordered = tuple(values[slot.name] for slot in self.signature.parameters(outputs=True))
        implicit = {name: value for name, value in symbols.items() if name not in values}
        return ordered, implicit, created

    def __call__(self, *inputs, **bindings):
        """Allocate the declared outputs, launch, and return one Buffer or a tuple of them."""
        ordered, dimensions, created = self.prepare(*inputs, **bindings)
        try:
            self.launch(*ordered, **dimensions)
        except BaseException:
            for buffer in created.values():
                buffer.release()
            raise
        results = tuple(created[name] for name in self.signature.outputs)
        return results[0] if len(results) == 1 else results
