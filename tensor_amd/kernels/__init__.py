"""Hand-written HIP kernels shipped as `hip` executable bundles (``<name>.tbin`` next to
their source), built by ``tensor_amd.build`` and loaded with ``Device.load(path)``.

Each entry gives the kernel's bundle manifest fields: its entry point, frontend
arguments (shapes over dimension symbols), kernel ABI order and launch geometry.
"""

from __future__ import annotations

from pathlib import Path

DIRECTORY = Path(__file__).resolve().parent


def _ceil_div(value, divisor):
    return {"op": "floordiv", "args": [{"op": "add", "args": [value, divisor - 1]}, divisor]}


BUNDLES = {
    # out = silu(gate) * up over [M, N] fp16: 8 elements per thread, 256 threads per workgroup
    "swiglu": {
        "entrypoint": "tensor_swiglu_f16",
        "symbols": {"M": "uint32", "N": "uint32"},
        "arguments": [
            {"kind": "buffer", "name": "gate", "dtype": "float16", "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
            {"kind": "buffer", "name": "up", "dtype": "float16", "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
            {"kind": "buffer", "name": "out", "dtype": "float16", "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
        ],
        "abi": [
            {"kind": "buffer", "name": "gate", "dtype": "float16"},
            {"kind": "buffer", "name": "up", "dtype": "float16"},
            {"kind": "buffer", "name": "out", "dtype": "float16"},
            {"kind": "scalar", "name": "M", "dtype": "uint32"},
            {"kind": "scalar", "name": "N", "dtype": "uint32"},
        ],
        "outputs": ["out"],
        "launch": {
            "grid": [_ceil_div({"op": "mul", "args": [{"var": "M"}, {"var": "N"}]}, 2048), 1, 1],
            "block": [256, 1, 1],
            "shared_memory_bytes": 0,
        },
        "op_set": ["swiglu"],
    },
}


def bundle_path(name: str) -> Path:
    """Path of a built bundle (raises if the name is unknown)."""
    if name not in BUNDLES:
        raise KeyError(f"unknown kernel bundle {name!r}")
    return DIRECTORY / f"{name}.tbin"
