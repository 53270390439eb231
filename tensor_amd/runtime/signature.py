"""Executable signatures: argument slots, symbolic shapes and launch geometry.

A manifest (the reference's executable schema, src/tensor/runtime/executable.py:87-149 and
signature.py:137-200) lists an executable's arguments -- buffers and scalars with their dtypes
-- and gives every buffer extent as an integer, a symbol ``{"var": "K"}`` or an integer
expression ``{"op": "mul", "args": [a, b]}`` / ``{"cast": "int32", "value": e}``.

``Signature`` compiles those expressions into closures once, when an executable is loaded:
binding a call then runs the closures instead of walking JSON, symbols are taken from the
extents that name them directly, every other extent is checked against its expression, and
scalars are range-checked before any ctypes value exists (ctypes would wrap them silently).
Nothing here calls ``eval``.
"""

from __future__ import annotations

import ctypes
import math
import numbers
import operator

import numpy as np

SCALAR_TYPES = {
    "bool": ctypes.c_bool, "int8": ctypes.c_int8, "int16": ctypes.c_int16, "int32": ctypes.c_int32,
    "int64": ctypes.c_int64, "uint8": ctypes.c_uint8, "uint16": ctypes.c_uint16, "uint32": ctypes.c_uint32,
    "uint64": ctypes.c_uint64, "float32": ctypes.c_float, "float64": ctypes.c_double,
}
# integer dtype -> inclusive (low, high) range
_RANGES = {name: (int(np.iinfo(name).min), int(np.iinfo(name).max))
           for name in SCALAR_TYPES if name not in ("bool", "float32", "float64")}
INTEGER_TYPES = frozenset(_RANGES)
_EXPRESSION_RANGE = _RANGES["int64"]


def buffer_argument(descriptor: dict) -> bool:
    """Arguments are buffers unless the manifest marks them ``"kind": "scalar"``."""
    return descriptor.get("kind", "buffer") == "buffer"


def scalar_value(value, dtype: str, name: str):
    """The canonical Python value of a scalar argument, or ValueError when it does not fit."""
    if dtype == "bool":
        if type(value) is not bool:
            raise ValueError(f"{name} needs a bool")
        return value
    if dtype in _RANGES:
        if isinstance(value, bool) or not isinstance(value, numbers.Integral):
            raise ValueError(f"{name} needs an integer {dtype}")
        low, high = _RANGES[dtype]
        if not low <= int(value) <= high:
            raise ValueError(f"{name} is outside the {dtype} range [{low}, {high}]")
        return int(value)
    if dtype not in SCALAR_TYPES:
        raise ValueError(f"{name}: unsupported scalar dtype {dtype}")
    if isinstance(value, bool) or not isinstance(value, numbers.Real):
        raise ValueError(f"{name} needs a real {dtype}")
    try:
        as_float = float(value)
    except OverflowError:
        as_float = math.inf
    stored = SCALAR_TYPES[dtype](as_float).value
    if not (math.isfinite(as_float) and math.isfinite(stored)):
        raise ValueError(f"{name} must be finite and representable as {dtype}")
    return stored


# ------------------------------------------------------------ expressions --

def _checked(operation):
    def apply(left, right):
        if operation in (operator.floordiv, operator.mod) and right == 0:
            raise ValueError("division by zero in a shape expression")
        result = operation(left, right)
        if not _EXPRESSION_RANGE[0] <= result <= _EXPRESSION_RANGE[1]:
            raise ValueError("shape expression overflows int64")
        return result
    return apply


_OPERATIONS = {"add": _checked(operator.add), "sub": _checked(operator.sub), "mul": _checked(operator.mul),
               "floordiv": _checked(operator.floordiv), "floormod": _checked(operator.mod),
               "min": _checked(min), "max": _checked(max)}


def _range_cast(value, dtype):
    return scalar_value(value, dtype, "dimension cast")


def compile_expression(tree, operations=None, cast=_range_cast):
    """A closure ``symbols -> int`` for one integer expression tree.  ``operations`` maps the
    operator names to two-argument functions (default: int64-checked integer arithmetic) and
    ``cast(value, dtype)`` applies a cast node, so the same trees also compile over other
    integer types (PyTorch's symbolic sizes)."""
    operations = _OPERATIONS if operations is None else operations
    if type(tree) is int:
        return lambda symbols: tree
    if not isinstance(tree, dict):
        raise ValueError(f"invalid shape expression {tree!r}")
    keys = set(tree)
    if keys == {"var"}:
        name = tree["var"]

        def symbol(symbols):
            try:
                return symbols[name]
            except KeyError:
                raise ValueError(f"dimension {name} is not bound; pass a buffer that fixes it or {name}=VALUE") \
                    from None
        return symbol
    if keys == {"cast", "value"}:
        inner, dtype = compile_expression(tree["value"], operations, cast), tree["cast"]
        return lambda symbols: cast(inner(symbols), dtype)
    if keys == {"op", "args"} and tree["op"] in operations and len(tree["args"]) == 2:
        operation = operations[tree["op"]]
        left, right = (compile_expression(arg, operations, cast) for arg in tree["args"])
        return lambda symbols: operation(left(symbols), right(symbols))
    raise ValueError(f"invalid shape expression {tree!r}")


def evaluate(tree, symbols: dict) -> int:
    return compile_expression(tree)(symbols)


# -------------------------------------------------------------- signature --

class Slot:
    """One manifest argument: name, kind, dtype and, for buffers, compiled extents."""

    __slots__ = ("name", "buffer", "dtype", "extents", "symbols", "alignment", "rank")

    def __init__(self, descriptor: dict):
        self.name, self.dtype = descriptor["name"], str(descriptor["dtype"])
        self.buffer = buffer_argument(descriptor)
        shape = descriptor.get("shape", ()) if self.buffer else ()
        self.rank = len(shape)
        self.extents = tuple(compile_expression(extent) for extent in shape)
        # the symbol an extent names directly (None for constants and expressions)
        self.symbols = tuple(extent["var"] if isinstance(extent, dict) and set(extent) == {"var"} else None
                             for extent in shape)
        self.alignment = int(descriptor.get("alignment", 256))

    def shape(self, symbols: dict) -> tuple:
        shape = tuple(extent(symbols) for extent in self.extents)
        if any(extent < 1 for extent in shape):
            raise ValueError(f"{self.name}: buffer extents must be positive, got {list(shape)}")
        return shape


class Signature:
    """The compiled form of a manifest's arguments, symbols, limits and launch geometry."""

    def __init__(self, manifest: dict):
        self.slots = [Slot(d) for d in manifest["arguments"]]
        self.by_name = {slot.name: slot for slot in self.slots}
        self.symbol_types = dict(manifest.get("symbols", {}))
        self.domains = {k: tuple(v) for k, v in manifest.get("shape_domain", {}).items()}
        self.divisors = dict(manifest.get("shape_divisors", {}))
        self.constants = dict(manifest.get("constants", {}))
        self.outputs = tuple(manifest.get("outputs", ()))
        launch = manifest["launch"]
        self._grid = tuple(compile_expression(v) for v in launch["grid"])
        self._block = tuple(compile_expression(v) for v in launch["block"])
        self._shared = compile_expression(launch["shared_memory_bytes"])
        # ABI order (defaults to the argument order)
        self.abi = [(d["name"], str(d["dtype"]), buffer_argument(d))
                    for d in manifest.get("abi", manifest["arguments"])]

    def parameters(self, *, outputs: bool = True) -> list:
        """Slots a caller supplies: every argument but the constants (and outputs, if asked)."""
        return [s for s in self.slots
                if s.name not in self.constants and (outputs or s.name not in self.outputs)]

    def bind(self, supplied: dict, dimensions: dict | None = None):
        """Derive the symbols from ``supplied`` buffers and scalars (plus explicit ``dimensions``),
        check every buffer against its declared shape and dtype, and return ``(symbols,
        values)`` with scalars canonicalised."""
        dimensions = dimensions or {}
        stray = set(dimensions) - set(self.symbol_types)
        if stray:
            raise ValueError(f"unknown dimensions: {sorted(stray)}")
        symbols = {name: scalar_value(value, self.symbol_types[name], name) for name, value in dimensions.items()}
        values = dict(supplied)

        def fix(symbol, value, where):
            known = symbols.setdefault(symbol, value)
            if known != value:
                raise ValueError(f"{where}: dimension {symbol} is {value}, but {known} was bound before")

        for slot in self.slots:
            if slot.name not in values:
                continue
            value = values[slot.name]
            if not slot.buffer:
                values[slot.name] = scalar_value(value, slot.dtype, slot.name)
                if slot.name in self.symbol_types:
                    fix(slot.name, values[slot.name], slot.name)
                continue
            shape, dtype = getattr(value, "shape", None), getattr(value, "dtype", None)
            if shape is None or dtype is None:
                raise TypeError(f"{slot.name} must be a buffer with a shape and a dtype")
            if len(shape) != slot.rank or str(dtype) != slot.dtype:
                raise ValueError(f"{slot.name}: expected a rank-{slot.rank} {slot.dtype} buffer, "
                                 f"got shape {tuple(shape)} {dtype}")
            for symbol, extent in zip(slot.symbols, shape):
                if symbol is not None:
                    fix(symbol, scalar_value(extent, self.symbol_types[symbol], symbol), slot.name)
        for slot in self.slots:
            if slot.buffer and slot.name in values:
                wanted = slot.shape(symbols)
                if tuple(values[slot.name].shape) != wanted:
                    raise ValueError(f"{slot.name}: expected shape {list(wanted)} {slot.dtype}, "
                                     f"got {list(values[slot.name].shape)}")
        for name, (low, high) in self.domains.items():
            if name in symbols and not low <= symbols[name] <= high:
                raise ValueError(f"dimension {name}={symbols[name]} is outside [{low}, {high}]")
        for name, divisor in self.divisors.items():
            if name in symbols and symbols[name] % divisor:
                raise ValueError(f"dimension {name}={symbols[name]} must be a multiple of {divisor}")
        return symbols, values

    def launch(self, symbols: dict) -> dict:
        grid = [f(symbols) for f in self._grid]
        block = [f(symbols) for f in self._block]
        shared = self._shared(symbols)
        if any(not 1 <= v < 1 << 31 for v in grid + block):
            raise ValueError("launch grid and block extents must be positive int32")
        if math.prod(block) > 1024:
            raise ValueError("launch block exceeds 1024 threads")
        if not 0 <= shared < 1 << 31:
            raise ValueError("invalid dynamic shared memory size")
        return {"grid": grid, "block": block, "shared_memory_bytes": shared}


def bind_shapes(manifest: dict, supplied: dict, dimensions: dict | None = None):
    """``Signature(manifest).bind(...)`` for callers that hold a manifest only."""
    return Signature(manifest).bind(supplied, dimensions)


def resolve_shape(shape, symbols: dict) -> tuple:
    result = tuple(compile_expression(extent)(symbols) for extent in shape)
    if any(extent < 1 for extent in result):
        raise ValueError(f"buffer extents must be positive, got {list(result)}")
    return result


def resolve_launch(launch: dict, symbols: dict) -> dict:
    return Signature({"arguments": [], "launch": launch}).launch(symbols)
