"""ORACLE — test infrastructure only.

Never imported by the product package (``tensor_amd``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module or load ``liboracle.so``, and only as the checker.

Two restatements of the reference's GGUF decoding live side by side:

* this NumPy module evaluates the reference's per-element index formulas
  (``benchmarks/kernels/showcase/triton_kernels.py:134-181``) over whole index
  grids, exactly as the Triton ``decode_ggml`` does for a tile;
* ``gguf_ref.c`` (built into ``liboracle.so``) walks every block sub-block by
  sub-block, the way the block is laid out.

The tests require both to agree bit for bit, and pin both with independent
encoders, exhaustive scale/min packing and closed forms.

Q8_0 does not appear in the reference's code (``research/plans/v1-benchmarks.md:301``
names it); it follows the public GGML definition: fp16 ``d`` then 32 int8,
``y = d * q``.  Q4_1, Q5_0, Q5_1, Q2_K, Q3_K and Q5_K (the plan's "other K-quants
and basic formats", ``research/plans/v1-benchmarks.md:297-300``) likewise follow the
public GGML block definitions; the C decoders list their layouts.

Product conventions: ``out[m, n] = sum_k x[m, k] * W[n, k]``
(``triton_kernels.py:199-211``).  Decode numerics use fp32 operands
(``benchmark.py:466-472``); prefill uses fp16-rounded operands
(``benchmark.py:473-477``).  Relative L2 is ``|a - e| / max(|e|, 1e-12)``
(``benchmarks/kernels/showcase/external_baselines.py:49-62``).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
# The other GGML encodings: public GGML block definitions, no reference code.
Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K = 3, 6, 7, 10, 11, 13
# GGML type id -> (elements per block, bytes per block)
GEOMETRY = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210),
            Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q2_K: (256, 84), Q3_K: (256, 110),
            Q5_K: (256, 176)}


def _half(raw: np.ndarray, offset: np.ndarray) -> np.ndarray:
    """fp16 at byte offsets (little-endian), widened exactly to fp32."""
    bits = raw[offset].astype(np.uint16) | (raw[offset + 1].astype(np.uint16) << 8)
    return bits.view(np.float16).astype(np.float32)


def dequantize(raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
    """Decode an ``[n, k]`` weight from raw GGML row-major blocks to fp32.

    Follows ``triton_kernels.py:134-181`` element by element: ``rows`` and
    ``channels`` are full index grids and every field is gathered per element.
    """
    qk, block = GEOMETRY[ggml_type]
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if k % qk or raw.size < n * (k // qk) * block:
        raise ValueError("raw buffer does not hold an [n, k] matrix of this type")
    rows = np.arange(n, dtype=np.int64)[:, None]
    channels = np.arange(k, dtype=np.int64)[None, :]
    base = rows * (k // qk * block) + channels // qk * block
    if ggml_type == Q4_0:  # triton_kernels.py:135-142
        scale = _half(raw, base)
        byte = raw[base + 2 + channels % 16].astype(np.int32)
        val = ((byte >> (channels % 32 // 16 * 4)) & 15) - 8
        return (val.astype(np.float32) * scale).astype(np.float32)
    if ggml_type == Q8_0:  # public GGML block_q8_0
        scale = _half(raw, base)
        val = raw[base + 2 + channels % 32].view(np.int8).astype(np.float32)
        return (scale * val).astype(np.float32)
    if ggml_type == Q4_K:  # triton_kernels.py:143-162
        local = channels % 256
        group = local // 32
        d = _half(raw, base)
        dm = _half(raw, base + 2)
        sc0 = raw[base + 4 + group % 4].astype(np.int32)
        sc1 = raw[base + 8 + group % 4].astype(np.int32)
        sc2 = raw[base + 12 + group % 4].astype(np.int32)
        sc = np.where(group < 4, sc0 & 63, (sc2 & 15) | ((sc0 >> 6) << 4))
        mn = np.where(group < 4, sc1 & 63, (sc2 >> 4) | ((sc1 >> 6) << 4))
        byte = raw[base + 16 + local // 64 * 32 + local % 32].astype(np.int32)
        val = (byte >> (local % 64 // 32 * 4)) & 15
        # d*sc*val is exact in fp32 and so is dm*mn; the subtraction rounds once.
        main = (d * sc.astype(np.float32)) * val.astype(np.float32)
        return (main - dm * mn.astype(np.float32)).astype(np.float32)
    if ggml_type == Q6_K:  # triton_kernels.py:163-180
        local = channels % 256
        half = local // 128
        lane = local % 32
        quarter = local % 128 // 32
        lo = raw[base + half * 64 + lane + (quarter % 2) * 32].astype(np.int32)
        hi = raw[base + 128 + half * 32 + lane].astype(np.int32)
        val = ((lo >> (quarter // 2 * 4)) & 15) | (((hi >> (quarter * 2)) & 3) << 4)
        sc = raw[base + 192 + local // 16].view(np.int8).astype(np.float32)
        d = _half(raw, base + 208)
        return (((val - 32).astype(np.float32) * sc) * d).astype(np.float32)
    if ggml_type in (Q4_1, Q5_0, Q5_1):  # 32-element blocks: nibble j and j + 16 share byte j
        d = _half(raw, base)
        lane = channels % 32
        tail = base + (2 if ggml_type == Q5_0 else 4)
        if ggml_type == Q4_1:
            byte = raw[tail + lane % 16].astype(np.int32)
            val = (byte >> (lane // 16 * 4)) & 15
            return (val.astype(np.float32) * d + _half(raw, base + 2)).astype(np.float32)
        byte = raw[tail + 4 + lane % 16].astype(np.int32)
        high = (raw[tail + lane // 8].astype(np.int32) >> (lane % 8)) & 1  # bit `lane` of qh
        val = ((byte >> (lane // 16 * 4)) & 15) | (high << 4)
        if ggml_type == Q5_0:
            return ((val - 16).astype(np.float32) * d).astype(np.float32)
        return (val.astype(np.float32) * d + _half(raw, base + 2)).astype(np.float32)
    if ggml_type == Q2_K:
        local = channels % 256
        sc = raw[base + local // 16].astype(np.int32)
        code = (raw[base + 16 + local // 128 * 32 + local % 32].astype(np.int32) >> (local % 128 // 32 * 2)) & 3
        d, dmin = _half(raw, base + 80), _half(raw, base + 82)
        main = (d * (sc & 15).astype(np.float32)) * code.astype(np.float32)
        return (main - dmin * (sc >> 4).astype(np.float32)).astype(np.float32)
    if ggml_type == Q3_K:
        local = channels % 256
        index = local // 16
        low = np.where(index < 8, raw[base + 96 + index % 8] & 15, raw[base + 96 + index % 8] >> 4).astype(np.int32)
        high = (raw[base + 104 + index % 4].astype(np.int32) >> (index // 4 * 2)) & 3
        scale = (low | (high << 4)) - 32
        code = (raw[base + 32 + local // 128 * 32 + local % 32].astype(np.int32) >> (local % 128 // 32 * 2)) & 3
        plane = local // 128 * 4 + local % 128 // 32
        keep = (raw[base + local % 32].astype(np.int32) >> plane) & 1
        val = code - np.where(keep == 1, 0, 4)
        d = _half(raw, base + 108)
        return ((d * scale.astype(np.float32)) * val.astype(np.float32)).astype(np.float32)
    if ggml_type == Q5_K:
        local = channels % 256
        group = local // 32
        d, dm = _half(raw, base), _half(raw, base + 2)
        sc0 = raw[base + 4 + group % 4].astype(np.int32)
        sc1 = raw[base + 8 + group % 4].astype(np.int32)
        sc2 = raw[base + 12 + group % 4].astype(np.int32)
        sc = np.where(group < 4, sc0 & 63, (sc2 & 15) | ((sc0 >> 6) << 4))
        mn = np.where(group < 4, sc1 & 63, (sc2 >> 4) | ((sc1 >> 6) << 4))
        byte = raw[base + 48 + local // 64 * 32 + local % 32].astype(np.int32)
        high = (raw[base + 16 + local % 32].astype(np.int32) >> group) & 1
        val = ((byte >> (local % 64 // 32 * 4)) & 15) | (high << 4)
        main = (d * sc.astype(np.float32)) * val.astype(np.float32)
        return (main - dm * mn.astype(np.float32)).astype(np.float32)
    raise ValueError(f"unsupported GGML type {ggml_type}")


def gemv_reference(x: np.ndarray, raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
    """Decode-path oracle: fp32 operands, accumulated in fp64 (benchmark.py:466-472)."""
    w = dequantize(raw, ggml_type, n, k).astype(np.float64)
    return np.asarray(x, dtype=np.float32).astype(np.float64).reshape(-1, k) @ w.T


def gemm_reference(x: np.ndarray, raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
    """Prefill oracle: fp16-rounded x and W, accumulated in fp64 (benchmark.py:473-477)."""
    w = dequantize(raw, ggml_type, n, k).astype(np.float16).astype(np.float64)
    xr = np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float64)
    return xr.reshape(-1, k) @ w.T


def silu(g: np.ndarray) -> np.ndarray:
    """g / (1 + exp(-g)) in fp64, the reference's SwiGLU gate
    (src/tensor/compiler/webgpu/schedules/packed_integer.py:204-205)."""
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


def swiglu_reference(x: np.ndarray, raw_gate: np.ndarray, raw_up: np.ndarray, ggml_type: int, n: int,
                     k: int) -> np.ndarray:
    """Gate / up pair with the SwiGLU epilogue: silu(x W_gate^T) * (x W_up^T), both
    products the decode oracle's (fp32 operands, fp64 sums), the epilogue in fp64
    (packed_integer.py:204-205 applies it to the two fp32 accumulators)."""
    return silu(gemv_reference(x, raw_gate, ggml_type, n, k)) * gemv_reference(x, raw_up, ggml_type, n, k)


def relative_l2(actual: np.ndarray, expected: np.ndarray) -> float:
    """external_baselines.py:49-62: |a - e|_2 / max(|e|_2, 1e-12)."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-12))


# ------------------------------------------------------------ C oracle -----


class COracle:
    """ctypes view of liboracle.so (gguf_ref.c)."""

    def __init__(self, path: Path = LIBRARY):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(path))
        lib.oracle_dequantize.argtypes = [
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
        ]
        lib.oracle_dequantize.restype = ctypes.c_int
        lib.oracle_linear.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ]
        lib.oracle_linear.restype = ctypes.c_int
        lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        lib.oracle_half_to_float.restype = ctypes.c_float
        lib.oracle_float_to_half.argtypes = [ctypes.c_float]
        lib.oracle_float_to_half.restype = ctypes.c_uint16
        lib.oracle_set_threads.argtypes = [ctypes.c_int]
        lib.oracle_max_threads.restype = ctypes.c_int
        self.lib = lib
        self.entry = lib.tensor_gguf_gemv_cpu_v1       # decode numerics (fp32 operands)
        self.gemm_entry = lib.tensor_gguf_gemm_cpu_v1  # prefill numerics (fp16 operands)

    def set_threads(self, threads: int) -> None:
        self.lib.oracle_set_threads(int(threads))

    def dequantize(self, raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.empty((n, k), dtype=np.float32)
        if self.lib.oracle_dequantize(ggml_type, raw.ctypes.data, n, k, out.ctypes.data):
            raise ValueError("oracle_dequantize rejected its arguments")
        return out

    def linear(self, x: np.ndarray, raw: np.ndarray, ggml_type: int, n: int, k: int,
               *, prefill: bool = False, out_dtype=np.float32) -> np.ndarray:
        x = np.ascontiguousarray(x)
        if x.dtype not in (np.float16, np.float32):
            raise TypeError("x must be fp16 or fp32")
        m = x.size // k
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.empty((m, n), dtype=out_dtype)
        status = self.lib.oracle_linear(
            ggml_type, int(prefill), x.ctypes.data, int(x.dtype == np.float16),
            raw.ctypes.data, out.ctypes.data, int(out.dtype == np.float16), m, n, k,
        )
        if status:
            raise ValueError(f"oracle_linear failed ({status})")
        return out


def c_oracle() -> COracle:
    return COracle()


def build(verbose: bool = False) -> Path:
    """Compile gguf_ref.c into liboracle.so (gcc, OpenMP)."""
    import subprocess

    cmd = [
        os.environ.get("CC", "gcc"), "-O2", "-fPIC", "-shared", "-fopenmp", "-std=c11",
        f"-I{HERE.parent / 'include'}", str(HERE / "gguf_ref.c"), "-o", str(LIBRARY) + ".tmp", "-lm",
    ]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(str(LIBRARY) + ".tmp", LIBRARY)
    return LIBRARY
