"""A HIP provider executable as a PyTorch operator.

Same surface as packages/tensor-torch/src/tensor_torch/kernel.py:15-98 and
registration.py:10-73: ``metadata`` / ``fake`` / ``raw`` / ``prepare`` /
``register`` / ``__call__`` / ``into``.  ``__call__`` goes through a
``torch.library`` custom operator with a fake (meta) implementation, so
torch.compile traces it with symbolic shapes; ``into`` is the registered
mutation form that writes caller-owned outputs.

Artifacts are the HIP provider's: a built-in GGUF kernel by name with its
options (``Kernel("gguf_linear", encoding="q4_k")``), a manifest dict, or a
``hip`` bundle by path.  Input buffers must be read-only in the kernel and
declared outputs completely written, never aliasing inputs (the functional
custom-operator contract); ``mutable_inputs`` names input buffers a kernel
without declared outputs writes, which ``raw`` and ``prepare`` launch.
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
from collections import OrderedDict
from itertools import count
from pathlib import Path

import torch

from tensor_amd.runtime.signature import buffer_argument
from tensor_amd.torch.launch import Prepared, _slots, launch, native_plan
from tensor_amd.torch.signatures import metadata

_operator_ids = count()


def _read_manifest(artifact, options):
    """(manifest, identity bytes, loader) for a kernel name, manifest dict or bundle path."""
    if isinstance(artifact, os.PathLike) or (isinstance(artifact, str) and os.path.isfile(artifact)):
        if options:
            raise ValueError("options apply only to kernels loaded by name")
        from tensor_amd.artifacts import read_artifact

        path = Path(artifact)
        manifest, _ = read_artifact(path)  # every member verified
        return manifest, path.read_bytes(), str(path)
    if isinstance(artifact, str):
        from tensor_amd.gguf.kernels import manifest as gguf_manifest

        manifest = gguf_manifest(artifact, **options)
        return manifest, json.dumps(manifest, sort_keys=True).encode(), manifest
    if isinstance(artifact, dict):
        if options:
            raise ValueError("options apply only to kernels loaded by name")
        return artifact, json.dumps(artifact, sort_keys=True).encode(), artifact
    raise TypeError("artifact must be a built-in kernel name, a manifest dict or a bundle path")


class Kernel:
    """A functional HIP executable with PyTorch-owned inputs and outputs."""

    def __init__(self, artifact, *, mutable_inputs=(), **options):
        self.artifact = artifact
        self.manifest, self._identity, self._loadable = _read_manifest(artifact, options)
        if self.manifest.get("provider") != "hip":
            raise ValueError("tensor_amd.torch runs HIP provider artifacts")
        names = self.manifest.get("outputs", [])
        if not names and not mutable_inputs:
            raise ValueError("functional kernels need declared outputs")
        constants = self.manifest.get("constants", {})
        self.inputs = [d for d in self.manifest["arguments"] if d["name"] not in names and d["name"] not in constants]
        self.outputs = [next(d for d in self.manifest["arguments"] if d["name"] == n) for n in names]
        self.mutable_inputs = tuple(mutable_inputs)
        if len(set(self.mutable_inputs)) != len(self.mutable_inputs) or set(self.mutable_inputs) - {
                d["name"] for d in self.inputs if buffer_argument(d)}:
            raise ValueError("mutable_inputs must name distinct input buffers")
        self._slots = _slots(self.manifest)
        self._executables: dict = {}
        self._prepared: OrderedDict = OrderedDict()
        # Rebinding native plans by input metadata, for kernels whose inputs are all tensors
        # (scalar values are not part of a plan's key).
        self._plans: dict | None = {} if all(buffer_argument(d) for d in self.inputs) else None
        self._lock = threading.RLock()
        self._op = None
        self._into_op = None

    def __repr__(self):
        return f"tensor_amd.torch.Kernel({self.manifest.get('name', self.manifest.get('entrypoint'))!r})"

    def _executable(self, device, ordinal):
        executable = self._executables.get(ordinal)
        if executable is None or not executable.device._open or executable.device is not device:
            executable = self._executables[ordinal] = device.load(self._loadable)
            self._prepared.clear()
            if self._plans is not None:
                self._plans.clear()
        return executable

    def metadata(self, args, *, symbolic=False):
        return metadata(self, args, symbolic=symbolic)

    def fake(self, args):
        outputs, device = self.metadata(args, symbolic=True)
        return [torch.empty(shape, dtype=dtype, device=device) for shape, dtype in outputs]

    def _launch(self, args, outputs, **options):
        return launch(self, args, outputs, **options)

    def _run(self, args):
        """Allocate the outputs and launch; a list of outputs.  Inputs whose metadata a
        native plan recorded go straight to it; others take the validated path, which
        records a plan for the next call."""
        plans = self._plans
        if plans is not None and args:
            key = tuple((t.shape, t.dtype, t.device) if isinstance(t, torch.Tensor) else None for t in args)
            entry = plans.get(key)
            if entry is not None and entry[1].device._open:
                result = entry[0](*args)
                if result is not None:
                    return [result] if len(self.outputs) == 1 else list(result)
        contract = self.metadata(args)
        outputs = [torch.empty(shape, dtype=dtype, device=contract[1]) for shape, dtype in contract[0]]
        executable, call, _, _ = self._launch(args, outputs, contract=contract, trusted_outputs=True)
        if plans is not None:
            plan = native_plan(self, executable, call, args, outputs, fixed=False)
            if plan is not None:
                if len(plans) >= 64:
                    plans.pop(next(iter(plans)))
                plans[key] = (plan, executable)
        return outputs

    def raw(self, *args):
        """Allocate the outputs and launch, bypassing the registered operator."""
        outputs = self._run(args)
        return outputs[0] if len(outputs) == 1 else tuple(outputs)

    def prepare(self, *args, outputs=None):
        """Bind fixed tensors and scalars once; the returned call launches on the current
        stream and never allocates.  Its outputs are ``.outputs``."""
        if outputs is None:
            contract = self.metadata(args)
            outputs = [torch.empty(shape, dtype=dtype, device=contract[1]) for shape, dtype in contract[0]]
        state = self._launch(args, list(outputs), enqueue=False)
        return Prepared(self, state, args, tuple(outputs))

    def register(self):
        return register(self)

    def __call__(self, *args):
        op = self._op or self.register()
        result = op([v for d, v in zip(self.inputs, args) if buffer_argument(d)],
                    [v for d, v in zip(self.inputs, args) if not buffer_argument(d)])
        return result[0] if len(result) == 1 else tuple(result)

    def into(self, *args, outputs):
        """Write caller-owned, disjoint outputs through the registered mutation operator."""
        if self._into_op is None:
            self.register()
        self._into_op([v for d, v in zip(self.inputs, args) if buffer_argument(d)],
                      [v for d, v in zip(self.inputs, args) if not buffer_argument(d)], list(outputs))


def register(kernel):
    """Register ``tensor_amd::kernel_<hash>_<n>`` and its ``_into`` mutation form."""
    if kernel.mutable_inputs:
        raise ValueError("kernels with mutable inputs cannot register as functional custom operators")
    if kernel._op is not None:
        return kernel._op
    # Each load is its own operator, even for the same artifact.
    name = f"kernel_{hashlib.sha256(kernel._identity).hexdigest()[:16]}_{next(_operator_ids)}"

    def unpack(tensors, scalars):
        tensors, scalars = iter(tensors), iter(scalars)
        return tuple(next(tensors) if buffer_argument(d) else next(scalars) for d in kernel.inputs)

    @torch.library.custom_op("tensor_amd::" + name, mutates_args=(),
                             schema="(Tensor[] tensors, Scalar[] scalars) -> Tensor[]")
    def op(tensors, scalars):
        return kernel._run(unpack(tensors, scalars))

    @op.register_fake
    def _(tensors, scalars):
        return kernel.fake(unpack(tensors, scalars))

    @torch.library.custom_op("tensor_amd::" + name + "_into", mutates_args={"outputs"},
                             schema="(Tensor[] tensors, Scalar[] scalars, Tensor(a!)[] outputs) -> ()")
    def into(tensors, scalars, outputs):
        kernel._launch(unpack(tensors, scalars), outputs)

    @into.register_fake
    def _(tensors, scalars, outputs):
        expected = kernel.fake(unpack(tensors, scalars))
        if len(expected) != len(outputs):
            raise ValueError("wrong output count")
        for want, out in zip(expected, outputs):
            if want.dtype != out.dtype or want.device != out.device or want.ndim != out.ndim or not out.is_contiguous():
                raise ValueError("output metadata mismatch")
            for lhs, rhs in zip(want.shape, out.shape):
                torch._check(lhs == rhs)

    kernel._op, kernel._into_op = op, into
    return op
