"""PyTorch argument checks and output metadata for a HIP kernel.

The behaviour is that of packages/tensor-torch/src/tensor_torch/signatures.py:12-86 (inputs are
contiguous tensors of one ROCm device; concrete shapes bind like a runtime call; symbolic shapes,
as torch.compile passes them to a fake kernel, are related through ``torch._check``).  The design
is this package's: a kernel's contract is compiled once, on first use, into a ``Contract`` that
holds the runtime ``Signature`` (concrete shapes take its binder as is) and, for symbolic shapes,
the same extent expressions compiled over SymInt arithmetic, so a fake call only walks prebuilt
lists.  The HIP manifests' ``shape_domain`` and ``shape_divisors`` hold on both paths.
"""

from __future__ import annotations

import operator

import torch

from tensor_amd.runtime.signature import Signature, buffer_argument, compile_expression

# SymInt arithmetic for the symbolic path; casts do not change a symbolic size
_SYMBOLIC = {"add": operator.add, "sub": operator.sub, "mul": operator.mul, "floordiv": operator.floordiv,
             "floormod": operator.mod, "min": torch.sym_min, "max": torch.sym_max}


def _symbolic(tree):
    return compile_expression(tree, _SYMBOLIC, cast=lambda value, dtype: value)


def torch_dtype(name: str):
    return getattr(torch, name)


class _Described:
    """What the binder reads of a tensor: its shape and its dtype's name."""

    __slots__ = ("shape", "dtype")

    def __init__(self, tensor):
        self.shape = tuple(tensor.shape)
        self.dtype = str(tensor.dtype).removeprefix("torch.")


class Contract:
    """One kernel's inputs and outputs, compiled for both binding paths."""

    def __init__(self, kernel):
        manifest = kernel.manifest
        self.signature = Signature(manifest)
        symbol_names = set(manifest.get("symbols", {}))
        # (name, is buffer) per input, in call order
        self.inputs = [(d["name"], buffer_argument(d)) for d in kernel.inputs]
        self.scalar_symbols = [name for name, is_buffer in self.inputs if not is_buffer and name in symbol_names]
        # per buffer input: name, rank, dtype name, and per axis the symbol it names directly
        # (or None) with the axis's symbolic extent
        self.buffers = []
        for d in kernel.inputs:
            if buffer_argument(d):
                axes = tuple((e["var"] if isinstance(e, dict) and set(e) == {"var"} else None, _symbolic(e))
                             for e in d["shape"])
                self.buffers.append((d["name"], len(axes), str(d["dtype"]), axes))
        self.outputs = [(self.signature.by_name[d["name"]], torch_dtype(d["dtype"]),
                         tuple(_symbolic(e) for e in d["shape"])) for d in kernel.outputs]

    def place(self, args):
        """(values by name for the binder, the tensors' device); tensors must be contiguous on
        one ROCm device."""
        if len(args) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs, received {len(args)}")
        values, devices = {}, []
        for (name, is_buffer), value in zip(self.inputs, args):
            if not is_buffer:
                values[name] = value
                continue
            if not isinstance(value, torch.Tensor):
                raise TypeError(f"{name} must be a PyTorch tensor")
            if value.device.type != "cuda" or not value.is_contiguous():
                raise ValueError("tensor_amd kernels require contiguous tensors on a ROCm device")
            if devices and value.device != devices[0]:
                raise ValueError("all inputs must be on the same ROCm device")
            devices.append(value.device)
            values[name] = _Described(value)
        if not devices:
            raise ValueError("a PyTorch kernel needs at least one tensor input")
        return values, devices[0]

    def concrete(self, values):
        symbols, _ = self.signature.bind(values, {})
        return [(slot.shape(symbols), dtype) for slot, dtype, _ in self.outputs]

    def symbolic(self, values):
        """Output (shape, dtype) over symbolic sizes: each symbol is taken from the first extent
        that names it, and every extent, domain and divisor becomes a ``torch._check``."""
        symbols = {name: values[name] for name in self.scalar_symbols}
        for name, rank, dtype, axes in self.buffers:
            described = values[name]
            if len(described.shape) != rank or described.dtype != dtype:
                raise ValueError(f"{name}: input rank or dtype mismatch")
            for (symbol, _), actual in zip(axes, described.shape):
                if symbol is not None:
                    symbols.setdefault(symbol, actual)
        for name, _, _, axes in self.buffers:
            for (_, extent), actual in zip(axes, values[name].shape):
                torch._check(extent(symbols) == actual, lambda name=name: f"{name}: shape mismatch")
        signature = self.signature
        for name, (low, high) in signature.domains.items():
            if name in symbols:
                torch._check(symbols[name] >= low, lambda name=name, low=low: f"dimension {name} is below {low}")
                torch._check(symbols[name] <= high, lambda name=name, high=high: f"dimension {name} is above {high}")
        for name, divisor in signature.divisors.items():
            if name in symbols:
                torch._check(symbols[name] % divisor == 0,
                             lambda name=name, divisor=divisor: f"dimension {name} must be a multiple of {divisor}")
        result = []
        for _, dtype, extents in self.outputs:
            shape = tuple(extent(symbols) for extent in extents)
            for extent in shape:
                torch._check(extent > 0)
            result.append((shape, dtype))
        return result


def contract(kernel) -> Contract:
    """The kernel's compiled contract (built on first use and kept on the kernel)."""
    compiled = getattr(kernel, "_contract", None)
    if compiled is None:
        compiled = kernel._contract = Contract(kernel)
    return compiled


def metadata(kernel, args, *, symbolic: bool = False):
    """([(shape, torch dtype)] of the outputs, device) for these inputs."""
    compiled = contract(kernel)
    values, device = compiled.place(args)
    return (compiled.symbolic(values) if symbolic else compiled.concrete(values)), device
