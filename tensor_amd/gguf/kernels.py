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
    "gguf_packed": "tensor_gguf_packed_v1",
    "gguf_gemv": "tensor_gguf_gemv_v1",
    "gguf_gemm": "tensor_gguf_gemm_v1",
    "gguf_linear": "tensor_gguf_linear_v1",
    "gguf_gemv_group": "tensor_gguf_gemv_group_v1",
    "gguf_gemm_group": "tensor_gguf_gemm_group_v1",
    "gguf_gemm_group_noalloc": "tensor_gguf_gemm_group_noalloc_v1",
    "gguf_gemm_group_plan": "tensor_gguf_gemm_group_plan_v1",
    "gguf_gemv_swiglu": "tensor_gguf_gemv_swiglu_v1",
    "gguf_gemv_variant": "tensor_gguf_gemv_variant_v1",
    "gguf_gemv_q8_1": "tensor_gguf_gemv_q8_1_v1",
    "gguf_dequant": "tensor_gguf_dequant_v1",
}
GEMV_GROUP_MAX = 3  # TENSOR_GGUF_GEMV_GROUP_MAX
Q8_1_TYPES = (2, 8, 12, 14)  # encodings of gguf_gemv_q8_1: Q4_0, Q8_0, Q4_K, Q6_K
OUT_DTYPES = ("float16", "float32")


def _row_bytes(code: int) -> dict:
    qk, block = GEOMETRY[code]
    return {"op": "mul", "args": [{"op": "floordiv", "args": [{"var": "K"}, qk]}, block]}


def _symbols(kernel: str, count: int | None) -> tuple:
    if kernel == "gguf_dequant":
        return ("N", "K")
    if kernel in ("gguf_gemv_group", "gguf_gemm_group_noalloc"):
        return ("M", "K", *(f"N{i}" for i in range(count)))
    if kernel in ("gguf_gemm_group", "gguf_gemm_group_plan"):
        return ("M", "K", *(f"N{i}" for i in range(count)), "W")
    return ("M", "N", "K")


GROUPS = ("gguf_gemv_group", "gguf_gemm_group", "gguf_gemm_group_noalloc", "gguf_gemm_group_plan")


def packed_manifest(encoding, m: int, n: int, k: int, *, x_dtype: str = "float32",
                    out_dtype: str = "float32") -> dict:
    """The showcase's own call form, specialised on (m, n, k) as AKAS specialises its kernels
    (``gguf(m, n, k, encoding)``, benchmarks/kernels/showcase/kernels.py:114-119): arguments
    ``[x, w, out]`` exactly as ``benchmark.py:460-464`` builds them -- flat fp32 ``x[M*K]``,
    the flat raw bytes of ``W``, flat fp32 ``out[M*N]`` -- with the GGML type and the shape
    fixed as constant scalars of ``tensor_gguf_packed_v1``.  M == 1 runs the decode GEMV on
    fp32 operands, M > 1 the prefill GEMM on fp16-rounded ones (the showcase's dispatch)."""
    code = ggml_type(encoding)
    qk, block = GEOMETRY[code]
    for name, value in (("m", m), ("n", n), ("k", k)):
        if type(value) is not int or not 1 <= value < 1 << 31:
            raise ValueError(f"{name} must be a positive int32")
    if k % qk:
        raise ValueError(f"k must be a multiple of {qk} for {NAMES[code]}")
    for name, dtype in (("x_dtype", x_dtype), ("out_dtype", out_dtype)):
        if str(dtype) not in OUT_DTYPES:
            raise ValueError(f"{name} must be one of {OUT_DTYPES}")
    arguments = [
        {"name": "x", "dtype": str(x_dtype), "shape": [m * k], "alignment": 16},
        {"name": "w", "dtype": "uint8", "shape": [n * (k // qk) * block], "alignment": 16},
        {"name": "out", "dtype": str(out_dtype), "shape": [m * n], "alignment": 16},
        {"name": "type", "dtype": "uint32", "kind": "scalar"},
        {"name": "m", "dtype": "uint32", "kind": "scalar"},
        {"name": "n", "dtype": "uint32", "kind": "scalar"},
        {"name": "k", "dtype": "uint32", "kind": "scalar"},
    ]
    return {
        "name": f"gguf_packed:{NAMES[code]}:{m}x{n}x{k}:{x_dtype}:{out_dtype}",
        "provider": "hip",
        "target": "gfx950",
        "entrypoint": ENTRYPOINTS["gguf_packed"],
        "runtime_abi": {"major": 1, "minor": 1,
                        "required_capabilities": ["contiguous", "executable_descriptors", "no_external_workspace",
                                                  "scalars"]},
        "arguments": arguments,
        "abi": [dict(item, kind=item.get("kind", "buffer")) for item in arguments],
        "outputs": ["out"],
        "constants": {"type": code, "m": m, "n": n, "k": k},
        "symbols": {},
        "launch": {"grid": [1, 1, 1], "block": [256, 1, 1], "shared_memory_bytes": 0},
        "ggml_type": code,
    }


def manifest(kernel: str, encoding, out_dtype: str | None = None, count: int | None = None, *,
             m: int | None = None, n: int | None = None, k: int | None = None,
             x_dtype: str | None = None) -> dict:
    """Build the manifest of one built-in GGUF executable.

    With ``m``, ``n`` and ``k`` (``gguf_linear`` or ``gguf_packed`` only) the executable is
    the showcase's shape-fixed packed form, ``packed_manifest``; ``x_dtype`` applies to it
    only.

    ``gguf_gemv_group`` takes ``count`` (1..3) weight matrices that share the
    activations: arguments ``[x, w0, out0, w1, out1, ..., type]`` with row
    counts ``N0, N1, ...``; ``gguf_gemm_group`` (the prefill GEMM of such a group,
    any M) adds a ``workspace`` uint8 buffer before ``type`` (its size
    ``Device.gemm_workspace`` tells); ``gguf_gemm_group_noalloc`` is the same GEMM
    without it, on the library's static scratch; ``gguf_gemm_group_plan`` is ``gguf_gemm_group``
    with two more scalars, ``tile`` and ``splits``, naming the plan it runs (plan sweeps: see
    ``Device.gemm_plan``); every other kernel takes no ``count``.
    ``gguf_gemv_swiglu`` takes ``[x, w_gate, w_up, out, type]`` and stores
    silu(x W_gate^T) * (x W_up^T).  ``gguf_gemv_q8_1`` (Q4_0, Q8_0, Q4_K, Q6_K; ``x_dtype``
    float32 by default, or float16) is the decode GEMV on Q8_1-quantized activations with
    integer dot products (GGML's path).  ``gguf_gemv_variant`` (Q4_K, 2 <= M <= 8) is ``gguf_gemv``
    with three more scalars, ``kernel``, ``a`` and ``b``, naming the multi-row plan it runs (plan
    sweeps: see ``Device.gemv_plan``).
    """
    if kernel not in ENTRYPOINTS:
        raise ValueError(f"unknown HIP kernel {kernel!r}; choose {', '.join(ENTRYPOINTS)}")
    shape = (m, n, k)
    if kernel == "gguf_packed" or any(v is not None for v in shape):
        if kernel not in ("gguf_linear", "gguf_packed") or any(v is None for v in shape) or count is not None:
            raise ValueError("m, n and k (all three) select the packed form of gguf_linear / gguf_packed")
        return packed_manifest(encoding, m, n, k, x_dtype=x_dtype or "float32", out_dtype=out_dtype or "float32")
    if x_dtype is not None and kernel != "gguf_gemv_q8_1":
        raise ValueError("x_dtype applies to the packed form (m, n, k) and gguf_gemv_q8_1 only")
    code = ggml_type(encoding)
    out_dtype = str(out_dtype or "float16")
    if out_dtype not in OUT_DTYPES:
        raise ValueError(f"out_dtype must be one of {OUT_DTYPES}")
    qk, _ = GEOMETRY[code]
    weight = {"name": "w", "dtype": "uint8", "shape": [{"var": "N"}, _row_bytes(code)], "alignment": 16}
    type_argument = {"name": "type", "dtype": "uint32", "kind": "scalar"}
    if (count is not None) != (kernel in GROUPS):
        raise ValueError(f"count applies to {' / '.join(GROUPS)} only, and they need it")
    if kernel in GROUPS:
        if not 1 <= int(count) <= GEMV_GROUP_MAX:
            raise ValueError(f"count must be in 1..{GEMV_GROUP_MAX}")
        count = int(count)
        arguments = [{"name": "x", "dtype": "float16", "shape": [{"var": "M"}, {"var": "K"}], "alignment": 16}]
        for i in range(count):
            arguments.append({"name": f"w{i}", "dtype": "uint8", "shape": [{"var": f"N{i}"}, _row_bytes(code)], "alignment": 16})
            arguments.append({"name": f"out{i}", "dtype": out_dtype, "shape": [{"var": "M"}, {"var": f"N{i}"}], "alignment": 16})
        if kernel in ("gguf_gemm_group", "gguf_gemm_group_plan"):
            arguments.append({"name": "workspace", "dtype": "uint8", "shape": [{"var": "W"}], "alignment": 256})
        arguments.append(type_argument)
        if kernel == "gguf_gemm_group_plan":  # the plan, supplied per call
            arguments += [{"name": "tile", "dtype": "uint32", "kind": "scalar"},
                          {"name": "splits", "dtype": "uint32", "kind": "scalar"}]
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
        x_type = "float16"
        if kernel == "gguf_gemv_q8_1":
            if code not in Q8_1_TYPES:
                raise ValueError("gguf_gemv_q8_1 runs Q4_0, Q8_0, Q4_K and Q6_K")
            x_type = str(x_dtype or "float32")
            if x_type not in OUT_DTYPES:
                raise ValueError(f"x_dtype must be one of {OUT_DTYPES}")
        arguments = [
            {"name": "x", "dtype": x_type, "shape": [{"var": "M"}, {"var": "K"}], "alignment": 16},
            weight,
            {"name": "out", "dtype": out_dtype, "shape": [{"var": "M"}, {"var": "N"}], "alignment": 16},
            type_argument,
        ]
        if kernel == "gguf_gemv_variant":  # the multi-row plan, supplied per call
            if code != ggml_type("q4_k"):
                raise ValueError("gguf_gemv_variant runs Q4_K only")
            arguments += [{"name": name, "dtype": "uint32", "kind": "scalar"} for name in ("kernel", "a", "b")]
    result = {
        "name": f"{kernel}:{NAMES[code]}:{out_dtype}" + (f":{count}" if kernel in GROUPS else ""),
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
        "outputs": [f"out{i}" for i in range(count)] if kernel in GROUPS else ["out"],
        "constants": {"type": code},
        "symbols": {name: "int32" for name in _symbols(kernel, count)},
        "shape_divisors": {"K": qk},
        # The entry point chooses its own launch geometry; these values are
        # what the descriptor carries, not what the kernel is launched with.
        "launch": {"grid": [1, 1, 1], "block": [256, 1, 1], "shared_memory_bytes": 0},
        "ggml_type": code,
    }
    if kernel in ("gguf_gemv", "gguf_gemv_group", "gguf_gemv_swiglu", "gguf_gemv_q8_1"):
        result["shape_domain"] = {"M": [1, GEMV_MAX_M]}
    if kernel == "gguf_gemv_variant":
        result["shape_domain"] = {"M": [2, GEMV_MAX_M]}
    return result
