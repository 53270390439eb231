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
    "gguf_dequant": "tensor_gguf_dequant_v1",
}
OUT_DTYPES = ("float16", "float32")


def _row_bytes(code: int) -> dict:
    qk, block = GEOMETRY[code]
    return {"op": "mul", "args": [{"op": "floordiv", "args": [{"var": "K"}, qk]}, block]}


def manifest(kernel: str, encoding, out_dtype: str = "float16") -> dict:
    """Build the manifest of one built-in GGUF executable."""
    if kernel not in ENTRYPOINTS:
        raise ValueError(f"unknown HIP kernel {kernel!r}; choose {', '.join(ENTRYPOINTS)}")
    code = ggml_type(encoding)
    out_dtype = str(out_dtype)
    if out_dtype not in OUT_DTYPES:
        raise ValueError(f"out_dtype must be one of {OUT_DTYPES}")
    qk, _ = GEOMETRY[code]
    weight = {"name": "w", "dtype": "uint8", "shape": [{"var": "N"}, _row_bytes(code)], "alignment": 16}
    type_argument = {"name": "type", "dtype": "uint32", "kind": "scalar"}
    if kernel == "gguf_dequant":
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
        "name": f"{kernel}:{NAMES[code]}:{out_dtype}",
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
        "outputs": ["out"],
        "constants": {"type": code},
        "symbols": {name: "int32" for name in (("N", "K") if kernel == "gguf_dequant" else ("M", "N", "K"))},
        "shape_divisors": {"K": qk},
        # The entry point chooses its own launch geometry; these values are
        # what the descriptor carries, not what the kernel is launched with.
        "launch": {"grid": [1, 1, 1], "block": [256, 1, 1], "shared_memory_bytes": 0},
        "ggml_type": code,
    }
    if kernel == "gguf_gemv":
        result["shape_domain"] = {"M": [1, GEMV_MAX_M]}
    return result
