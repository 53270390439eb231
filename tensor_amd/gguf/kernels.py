"""Manifests of the built-in GGUF executables of the HIP provider.

The reference describes every executable with a manifest (argument names,
dtypes, symbolic shapes, outputs, launch) inside a .tbin artifact and binds
calls against it (src/tensor/runtime/executable.py:87-149,
src/tensor/runtime/signature.py:137-200).  The HIP provider's GGUF kernels are
hand-written and ship inside libtensor_hip.so, so their manifests are built
here, specialised per GGML encoding and output dtype, and loaded with
``Device.load("gguf_linear", encoding="q4_k", out_dtype="float16")``.

Argument order is the showcase's ``[x, w, out]``
(benchmarks/kernels/showcase/benchmark.py:293-295, :460-464) followed by the
GGML type scalar, which the manifest fixes as a constant.
"""

from __future__ import annotations

from tensor_amd.gguf.quant import GEOMETRY, NAMES, ggml_type

GEMV_MAX_M = 8  # TENSOR_GGUF_GEMV_MAX_M

ENTRYPOINTS = {
    "gguf_gemv": "tensor_gguf_gemv_v1",
    "gguf_gemm": "tensor_gguf_gemm_v1",
    "gguf_linear": "tensor_gguf_linear_v1",
    "gguf_gemv_group": "tensor_gguf_gemv_group_v1",
    "gguf_gemv_swiglu": "tensor_gguf_gemv_swiglu_v1",
    "gguf_dequant": "tensor_gguf_dequant_v1",
}
GEMV_GROUP_MAX = 3  # TENSOR_GGUF_GEMV_GROUP_MAX
OUT_DTYPES = ("float16", "float32")


def _row_bytes(code: int) -> dict:
    qk, block = GEOMETRY[code]
    return {"op": "mul", "args": [{"op": "floordiv", "args": [{"var": "K"}, qk]}, block]}


def _symbols(kernel: str, count: int | None) -> tuple:
    if kernel == "gguf_dequant":
        return ("N", "K")
    if kernel == "gguf_gemv_group":
        return ("M", "K", *(f"N{i}" for i in range(count)))
    return ("M", "N", "K")


def manifest(kernel: str, encoding, out_dtype: str = "float16", count: int | None = None) -> dict:
    """Build the manifest of one built-in GGUF executable.

    ``gguf_gemv_group`` takes ``count`` (1..3) weight matrices that share the
    activations: arguments ``[x, w0, out0, w1, out1, ..., type]`` with row
    counts ``N0, N1, ...``; every other kernel takes no ``count``.
    ``gguf_gemv_swiglu`` takes ``[x, w_gate, w_up, out, type]`` and stores
    silu(x W_gate^T) * (x W_up^T).
    """
    if kernel not in ENTRYPOINTS:
        raise ValueError(f"unknown HIP kernel {kernel!r}; choose {', '.join(ENTRYPOINTS)}")
    code = ggml_type(encoding)
    out_dtype = str(out_dtype)
    if out_dtype not in OUT_DTYPES:
        raise ValueError(f"out_dtype must be one of {OUT_DTYPES}")
    qk, _ = GEOMETRY[code]
    weight = {"name": "w", "dtype": "uint8", "shape": [{"var": "N"}, _row_bytes(code)], "alignment": 16}
    type_argument = {"name": "type", "dtype": "uint32", "kind": "scalar"}
    if (count is not None) != (kernel == "gguf_gemv_group"):
        raise ValueError("count applies to gguf_gemv_group only, and gguf_gemv_group needs it")
    if kernel == "gguf_gemv_group":
        if not 1 <= int(count) <= GEMV_GROUP_MAX:
            raise ValueError(f"count must be in 1..{GEMV_GROUP_MAX}")
        count = int(count)
        arguments = [{"name": "x", "dtype": "float16", "shape": [{"var": "M"}, {"var": "K"}], "alignment": 16}]
        for i in range(count):
            arguments.append({"name": f"w{i}", "dtype": "uint8", "shape": [{"var": f"N{i}"}, _row_bytes(code)], "alignment": 16})
            arguments.append({"name": f"out{i}", "dtype": out_dtype, "shape": [{"var": "M"}, {"var": f"N{i}"}], "alignment": 16})
        arguments.append(type_argument)
    elif kernel == "gguf_gemv_swiglu":
        arguments = [
            {"name": "x", "dtype": "float16", "shape": [{"var": "M"}, {"var": "K"}], "alignment": 16},
            dict(weight, name="w_gate"),
            dict(weight, name="w_up"),
            {"name": "out", "dtype": out_dtype, "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
            type_argument,
        ]
    elif kernel == "gguf_dequant":
        arguments = [
            weight,
            {"name": "out", "dtype": out_dtype, "shape": [{"var": "N"}, {"var": "K"}], "alignment": 16},
            type_argument,
        ]
    else:
        arguments = [
            {"name": "x", "dtype": "float16", "shape": [{"var": "M"}, {"var": "K"}], "alignment": 16},
            weight,
            {"name": "out", "dtype": out_dtype, "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
            type_argument,
        ]
    result = {
        "name": f"{kernel}:{NAMES[code]}:{out_dtype}" + (f":{count}" if kernel == "gguf_gemv_group" else ""),
        "provider": "hip",
        "target": "gfx950",
        "entrypoint": ENTRYPOINTS[kernel],
        "runtime_abi": {
            "major": 1,
            "minor": 1,
            "required_capabilities": ["contiguous", "executable_descriptors", "no_external_workspace", "scalars"],
        },
        "arguments": arguments,
        "abi": [dict(item, kind=item.get("kind", "buffer")) for item in arguments],
        "outputs": [f"out{i}" for i in range(count)] if kernel == "gguf_gemv_group" else ["out"],
        "constants": {"type": code},
        "symbols": {name: "int32" for name in _symbols(kernel, count)},
        "shape_divisors": {"K": qk},
        # The entry point chooses its own launch geometry; these values are
        # what the descriptor carries, not what the kernel is launched with.
        "launch": {"grid": [1, 1, 1], "block": [256, 1, 1], "shared_memory_bytes": 0},
        "ggml_type": code,
    }
    if kernel in ("gguf_gemv", "gguf_gemv_group", "gguf_gemv_swiglu"):
        result["shape_domain"] = {"M": [1, GEMV_MAX_M]}
    return result
