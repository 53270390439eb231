"""Loaded executables: the reference's Executable surface (src/tensor/runtime/executable.py):
``launch``, ``bind`` (a retained ``BoundCall``), ``prepare`` (allocate the declared outputs),
``__call__`` (allocate, launch, return the outputs), ``descriptor``, ``workspace_requirements``,
``release`` and the context-manager protocol, with the same errors.

How this build organises it: the manifest is compiled once, at load, into a ``Signature`` and two
``_CallForm`` objects (the argument order and accepted names of calls that pass their outputs and
of calls that do not), and the provider's load products live in one ``_Loaded`` record, so a call
is matched by table lookups and a release is one state change.  Buffers are admitted through the
storage record they share with their views (one test, however deep the view chain).
"""

from __future__ import annotations

import ctypes as c
import math

from tensor_amd.runtime.abi import ABI_MAJOR, BoundCall, ExecutableDescriptor, WorkspaceRequirements
from tensor_amd.runtime.buffer import Buffer
from tensor_amd.runtime.signature import Signature

TENSOR_EXEC_ASYNC = 1


class _Loaded:
    """What the provider's load produced and the session it is valid in."""

    __slots__ = ("module", "function", "image", "generation", "released")

    def __init__(self, module, function, image, generation):
        self.module, self.function, self.image = module, function, image
        self.generation, self.released = generation, False


class _CallForm:
    """The names a call's values bind to, in call order, for one form of call."""

    __slots__ = ("order", "accepted", "symbols", "buffers")

    def __init__(self, signature: Signature, *, outputs: bool):
        slots = signature.parameters(outputs=outputs)
        self.order = tuple(slot.name for slot in slots)
        self.accepted = frozenset(self.order)
        self.symbols = frozenset(signature.symbol_types)
        self.buffers = tuple(slot for slot in slots if slot.buffer)

    def collect(self, arguments: tuple, keywords: dict):
        """(values by name, explicit dimensions) for positional and keyword arguments."""
        if len(arguments) > len(self.order):
            raise ValueError(f"kernel expects at most {len(self.order)} arguments, received {len(arguments)}")
        values = dict(zip(self.order, arguments))
        dimensions = {}
        for name, value in keywords.items():
            if name in values:
                raise ValueError(f"argument {name} supplied twice")
            target = values if name in self.accepted else dimensions if name in self.symbols else None
            if target is None:
                raise ValueError(f"unknown kernel argument {name}")
            target[name] = value
        if len(values) != len(self.order):
            raise ValueError(f"missing kernel arguments: {sorted(self.accepted.difference(values))}")
        return values, dimensions


class Executable:
    def __init__(self, device, manifest: dict, module, function, image):
        self.device, self.manifest = device, manifest
        self.signature = Signature(manifest)
        self._forms = {True: _CallForm(self.signature, outputs=True), False: _CallForm(self.signature, outputs=False)}
        self._loaded = _Loaded(module, function, image, device._generation)
        self._handle = device._registry.ticket()
        flags = TENSOR_EXEC_ASYNC if "async_launch" in device.capabilities else 0
        self._descriptor = ExecutableDescriptor(ABI_MAJOR, c.sizeof(ExecutableDescriptor), device.device_type,
                                                device.ordinal, device._session_id, self._handle,
                                                len(self.signature.abi), flags,
                                                WorkspaceRequirements(0, 1, device.device_type, 0, 0))
        device._executables[self._handle] = self

    module = property(lambda self: self._loaded.module)
    function = property(lambda self: self._loaded.function)
    _generation = property(lambda self: self._loaded.generation)
    _released = property(lambda self: self._loaded.released)

    def __repr__(self):
        return f"Executable({self.manifest.get('name', self.manifest.get('entrypoint'))})"

    # -- lifetime -------------------------------------------------------------
    def _fault(self):
        """Why this executable cannot be used now (None when it can); no native call."""
        device = self.device
        if not device._open:
            return "device session is closed"
        if self._loaded.generation != device._generation:
            return "executable belongs to a previous device session"
        if self._loaded.released:
            return "executable has been released"
        return None

    def _check(self) -> None:
        fault = self._fault()
        if fault:
            raise self.device.error(fault)

    @property
    def descriptor(self):
        self._check()
        return ExecutableDescriptor.from_buffer_copy(self._descriptor)

    def workspace_requirements(self):
        self._check()
        return WorkspaceRequirements.from_buffer_copy(self._descriptor.workspace)

    def release(self) -> None:
        if self._loaded.released:
            return
        self._check()
        self.device.synchronize()
        self._dispose()

    def _dispose(self) -> None:
        loaded = self._loaded
        if loaded.released:
            return
        self.device._unload_executable(self)
        self.device._executables.pop(self._handle, None)
        loaded.released = True
        loaded.module = loaded.function = loaded.image = None

    def __enter__(self):
        self._check()
        return self

    def __exit__(self, *exc):
        self.release()

    # -- calls ----------------------------------------------------------------
    def _admit(self, form: _CallForm, values: dict) -> None:
        """Every buffer of the call is a live Buffer of this session, suitably aligned."""
        for slot in form.buffers:
            buffer = values[slot.name]
            if not isinstance(buffer, Buffer):
                raise TypeError(f"{slot.name} must be a Tensor Buffer")
            if buffer.device is not self.device:
                raise ValueError(f"{slot.name} belongs to a different device session")
            if buffer._released or buffer._generation != self._loaded.generation:
                raise self.device.error("buffer has been released")
            if buffer.pointer % slot.alignment:
                raise ValueError(f"{slot.name} needs {slot.alignment}-byte pointer alignment")

    def _resolve(self, arguments: tuple, keywords: dict, *, outputs: bool):
        """(symbols, values) of a checked call: matched, admitted and bound to the signature."""
        form = self._forms[outputs]
        values, dimensions = form.collect(arguments, keywords)
        self._admit(form, values)
        return self.signature.bind(values, dimensions)

    def _launch_geometry(self, symbols: dict) -> dict:
        geometry = self.signature.launch(symbols)
        limits = self.device.limits
        for field in ("grid", "block"):
            if any(value > limit for value, limit in zip(geometry[field], limits[field])):
                raise ValueError(f"launch {field} exceeds this device's limits")
        threads = limits.get("threads")
        if threads is not None and math.prod(geometry["block"]) > threads:
            raise ValueError("launch thread count exceeds this device's limit")
        return geometry

    def bind(self, *arguments, **bindings) -> BoundCall:
        """Validate once and return a BoundCall for repeated, allocation-free submission.
        Bind again when shapes, scalars or storage change."""
        self._check()
        symbols, values = self._resolve(arguments, bindings, outputs=True)
        return BoundCall(self, values, symbols, self._launch_geometry(symbols), self.device.stream_descriptor())

    def launch(self, *arguments, **bindings) -> None:
        """Launch with every buffer argument, outputs included."""
        self.bind(*arguments, **bindings).launch()

    def prepare(self, *inputs, **bindings):
        """Allocate the declared outputs for these inputs without launching; returns the full
        argument tuple, the dimensions the inputs did not fix, and the new outputs by name."""
        self._check()
        if not self.signature.outputs:
            raise ValueError("artifact has no declared outputs; call launch with every buffer")
        symbols, values = self._resolve(inputs, bindings, outputs=False)
        created = _Outputs(self.device)
        with created:
            for name in self.signature.outputs:
                slot = self.signature.by_name[name]
                created.add(name, slot.shape(symbols), slot.dtype)
        values.update(created.buffers)
        ordered = tuple(values[name] for name in self._forms[True].order)
        implicit = {name: value for name, value in symbols.items() if name not in values}
        return ordered, implicit, dict(created.buffers)

    def __call__(self, *inputs, **bindings):
        """Allocate the declared outputs, launch, and return one Buffer or a tuple of them."""
        ordered, dimensions, created = self.prepare(*inputs, **bindings)
        outputs = _Outputs(self.device, created)
        with outputs:
            self.launch(*ordered, **dimensions)
        results = tuple(created[name] for name in self.signature.outputs)
        return results[0] if len(results) == 1 else results


class _Outputs:
    """Buffers allocated for a call, released again if the block that fills or uses them fails."""

    def __init__(self, device, buffers=None):
        self.device, self.buffers = device, dict(buffers or {})

    def add(self, name, shape, dtype) -> None:
        self.buffers[name] = self.device.empty(shape, dtype)

    def __enter__(self):
        return self

    def __exit__(self, kind, error, trace):
        if kind is not None:
            for buffer in self.buffers.values():
                buffer.release()
        return False
