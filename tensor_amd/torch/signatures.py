"""Validate PyTorch arguments and infer the declared outputs' shapes and dtypes.

Behaviour of packages/tensor-torch/src/tensor_torch/signatures.py:12-86:
buffer inputs are contiguous tensors of one ROCm device; concrete shapes go
through the runtime's binder, symbolic (fake) shapes through ``torch._check``
so that torch.compile can trace the operator with dynamic extents.  The HIP
manifests also carry ``shape_domain`` and ``shape_divisors``; both are checked
on either path.
"""

from __future__ import annotations

import operator

import torch

from tensor_amd.runtime.signature import bind_shapes, buffer_argument, resolve_shape

_SYMBOLIC = {
    "add": operator.add,
    "sub": operator.sub,
    "mul": operator.mul,
    "floordiv": operator.floordiv,
    "floormod": operator.mod,
    "min": lambda a, b: torch.sym_min(a, b),
    "max": lambda a, b: torch.sym_max(a, b),
}


class _Described:
    """What the binder reads of a tensor: its shape and its dtype's name."""

    def __init__(self, tensor):
        self.shape = tuple(tensor.shape)
        self.dtype = str(tensor.dtype).removeprefix("torch.")


def torch_dtype(name: str):
    return getattr(torch, name)


def metadata(kernel, args, *, symbolic: bool = False):
    """([(shape, torch dtype)] of the outputs, device) for these inputs."""
    if len(args) != len(kernel.inputs):
        raise ValueError(f"expected {len(kernel.inputs)} inputs, received {len(args)}")
    values, device = {}, None
    for descriptor, value in zip(kernel.inputs, args):
        if not buffer_argument(descriptor):
            values[descriptor["name"]] = value
            continue
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{descriptor['name']} must be a PyTorch tensor")
        if value.device.type != "cuda" or not value.is_contiguous():
            raise ValueError("tensor_amd kernels require contiguous tensors on a ROCm device")
        if device is not None and value.device != device:
            raise ValueError("all inputs must be on the same ROCm device")
        device = value.device
        values[descriptor["name"]] = _Described(value)
    if device is None:
        raise ValueError("a PyTorch kernel needs at least one tensor input")
    manifest = kernel.manifest
    if not symbolic:
        symbols, _ = bind_shapes(manifest, values, {})
        shapes = [resolve_shape(d["shape"], symbols) for d in kernel.outputs]
        return [(shape, torch_dtype(d["dtype"])) for shape, d in zip(shapes, kernel.outputs)], device

    symbols = {}
    for descriptor in kernel.inputs:
        value = values[descriptor["name"]]
        if buffer_argument(descriptor):
            if len(value.shape) != len(descriptor["shape"]) or value.dtype != descriptor["dtype"]:
                raise ValueError(f"{descriptor['name']}: input rank or dtype mismatch")
            for extent, actual in zip(descriptor["shape"], value.shape):
                if isinstance(extent, dict) and set(extent) == {"var"}:
                    name = extent["var"]
                    if name in symbols:
                        torch._check(symbols[name] == actual, lambda: f"dimension {name} mismatch")
                    else:
                        symbols[name] = actual
        elif descriptor["name"] in manifest.get("symbols", {}):
            symbols[descriptor["name"]] = value

    def evaluate(expression):
        if type(expression) is int:
            return expression
        if "var" in expression:
            return symbols[expression["var"]]
        if "cast" in expression:
            return evaluate(expression["value"])
        left, right = (evaluate(item) for item in expression["args"])
        return _SYMBOLIC[expression["op"]](left, right)

    for descriptor in kernel.inputs:
        if buffer_argument(descriptor):
            for extent, actual in zip(descriptor["shape"], values[descriptor["name"]].shape):
                torch._check(evaluate(extent) == actual, lambda: f"{descriptor['name']}: shape mismatch")
    for name, (low, high) in manifest.get("shape_domain", {}).items():
        if name in symbols:
            torch._check(symbols[name] >= low, lambda: f"dimension {name} is below {low}")
            torch._check(symbols[name] <= high, lambda: f"dimension {name} is above {high}")
    for name, divisor in manifest.get("shape_divisors", {}).items():
        if name in symbols:
            torch._check(symbols[name] % divisor == 0, lambda: f"dimension {name} must be a multiple of {divisor}")
    shapes = [tuple(evaluate(extent) for extent in d["shape"]) for d in kernel.outputs]
    for shape in shapes:
        for extent in shape:
            torch._check(extent > 0)
    return [(shape, torch_dtype(d["dtype"])) for shape, d in zip(shapes, kernel.outputs)], device
