"""Scalar, symbolic-shape and launch binding for executable manifests.

Behaviour follows the reference's provider-neutral binder
(src/tensor/runtime/signature.py:28-216): scalars are range-checked before a
ctypes value is built (ctypes would silently wrap), shapes may name symbols
(``{"var": "K"}``) or bounded integer expressions (``{"op": "mul", "args":
[...]}``), and no Python ``eval`` is ever used.
"""

from __future__ import annotations

import ctypes
import math
import numbers

SCALAR_TYPES = {
    "bool": ctypes.c_bool,
    "int8": ctypes.c_int8,
    "int16": ctypes.c_int16,
    "int32": ctypes.c_int32,
    "int64": ctypes.c_int64,
    "uint8": ctypes.c_uint8,
    "uint16": ctypes.c_uint16,
    "uint32": ctypes.c_uint32,
    "uint64": ctypes.c_uint64,
    "float32": ctypes.c_float,
    "float64": ctypes.c_double,
}
INTEGER_TYPES = frozenset(SCALAR_TYPES) - {"bool", "float32", "float64"}
OPERATIONS = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "floordiv": lambda a, b: a // b,
    "floormod": lambda a, b: a % b,
    "min": min,
    "max": max,
}
_INT64 = (-(1 << 63), (1 << 63) - 1)


def scalar_value(value, dtype: str, name: str):
    """Validate a Python scalar for ``dtype``; returns the canonical value."""
    if dtype not in SCALAR_TYPES:
        raise ValueError(f"{name}: unsupported scalar dtype {dtype}")
    if dtype == "bool":
        if not isinstance(value, bool):
            raise ValueError(f"{name} needs a bool")
        return value
    if dtype in INTEGER_TYPES:
        if isinstance(value, bool) or not isinstance(value, numbers.Integral):
            raise ValueError(f"{name} needs an integer {dtype}")
        value = int(value)
        bits = ctypes.sizeof(SCALAR_TYPES[dtype]) * 8
        signed = not dtype.startswith("u")
        low = -(1 << (bits - 1)) if signed else 0
        high = (1 << (bits - 1)) - 1 if signed else (1 << bits) - 1
        if not low <= value <= high:
            raise ValueError(f"{name} is outside the {dtype} range")
        return value
    if isinstance(value, bool) or not isinstance(value, numbers.Real):
        raise ValueError(f"{name} needs a real {dtype}")
    try:
        value = float(value)
    except OverflowError as exc:
        raise ValueError(f"{name} must be finite and fit {dtype}") from exc
    converted = SCALAR_TYPES[dtype](value).value
    if not (math.isfinite(value) and math.isfinite(converted)):
        raise ValueError(f"{name} must be finite and fit {dtype}")
    return converted


def evaluate(expression, symbols: dict) -> int:
    """Evaluate an integer expression tree against bound symbols."""
    if type(expression) is int:
        return expression
    if not isinstance(expression, dict):
        raise ValueError("invalid integer expression")
    if set(expression) == {"var"}:
        name = expression["var"]
        if name not in symbols:
            raise ValueError(f"cannot bind dimension {name}; supply a matching input or {name}=VALUE")
        return symbols[name]
    if set(expression) == {"cast", "value"}:
        return scalar_value(evaluate(expression["value"], symbols), expression["cast"], "dimension cast")
    if set(expression) != {"op", "args"} or expression["op"] not in OPERATIONS:
        raise ValueError("invalid integer expression operation")
    if len(expression["args"]) != 2:
        raise ValueError("integer expressions take two operands")
    left, right = (evaluate(value, symbols) for value in expression["args"])
    if expression["op"] in ("floordiv", "floormod") and right == 0:
        raise ValueError("division by zero in integer expression")
    result = OPERATIONS[expression["op"]](left, right)
    if not _INT64[0] <= result <= _INT64[1]:
        raise ValueError("integer expression overflow")
    return result


def buffer_argument(descriptor: dict) -> bool:
    return descriptor.get("kind", "buffer") == "buffer"


def resolve_shape(shape: list, symbols: dict) -> tuple:
    result = tuple(evaluate(value, symbols) for value in shape)
    if any(value < 1 for value in result):
        raise ValueError("buffer shape must contain positive extents")
    return result


def bind_shapes(manifest: dict, supplied: dict, dimensions: dict | None = None):
    """Bind direct symbols from buffer shapes, then check every buffer shape.

    Returns ``(symbols, values)`` with scalars canonicalised.
    """
    definitions = manifest.get("symbols", {})
    dimensions = dimensions or {}
    unknown = set(dimensions) - set(definitions)
    if unknown:
        raise ValueError(f"unknown dimensions: {sorted(unknown)}")
    bound = {name: scalar_value(value, definitions[name], name) for name, value in dimensions.items()}
    values = dict(supplied)

    def bind(symbol, value, where):
        if symbol in bound and bound[symbol] != value:
            raise ValueError(f"{where}: dimension {symbol} mismatch; expected {bound[symbol]}, received {value}")
        bound[symbol] = value

    for descriptor in manifest["arguments"]:
        name = descriptor["name"]
        if name not in values:
            continue
        value = values[name]
        if not buffer_argument(descriptor):
            values[name] = scalar_value(value, descriptor["dtype"], name)
            if name in definitions:
                bind(name, values[name], name)
            continue
        if not hasattr(value, "shape") or not hasattr(value, "dtype"):
            raise TypeError(f"{name} must be a buffer with shape and dtype")
        if len(value.shape) != len(descriptor["shape"]) or str(value.dtype) != descriptor["dtype"]:
            raise ValueError(f"{name} needs shape {descriptor['shape']} and dtype {descriptor['dtype']}")
        for extent, actual in zip(descriptor["shape"], value.shape):
            if isinstance(extent, dict) and set(extent) == {"var"}:
                symbol = extent["var"]
                bind(symbol, scalar_value(actual, definitions[symbol], symbol), name)
    for descriptor in manifest["arguments"]:
        name = descriptor["name"]
        if name in values and buffer_argument(descriptor):
            expected = resolve_shape(descriptor["shape"], bound)
            if tuple(values[name].shape) != expected:
                raise ValueError(f"{name} needs shape {list(expected)} and dtype {descriptor['dtype']}")
    for name, (low, high) in manifest.get("shape_domain", {}).items():
        if name in bound and not low <= bound[name] <= high:
            raise ValueError(f"dimension {name}={bound[name]} is outside [{low}, {high}]")
    for name, divisor in manifest.get("shape_divisors", {}).items():
        if name in bound and bound[name] % divisor:
            raise ValueError(f"dimension {name}={bound[name]} must be a multiple of {divisor}")
    return bound, values


def resolve_launch(launch: dict, symbols: dict) -> dict:
    result = {name: [evaluate(value, symbols) for value in launch[name]] for name in ("grid", "block")}
    result["shared_memory_bytes"] = evaluate(launch["shared_memory_bytes"], symbols)
    for name in ("grid", "block"):
        if any(value < 1 or value > (1 << 31) - 1 for value in result[name]):
            raise ValueError(f"launch {name} exceeds positive int32 dimensions")
    if math.prod(result["block"]) > 1024:
        raise ValueError("launch block exceeds 1024 threads")
    if not 0 <= result["shared_memory_bytes"] <= (1 << 31) - 1:
        raise ValueError("invalid shared memory size")
    return result
