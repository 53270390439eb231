"""Seeded inputs shared by the GPU parity tests and the benchmark checks."""

from __future__ import annotations

import numpy as np

from tensor_amd.gguf import quant as Q

SLAB_ROWS = 2048


def weight(n: int, k: int, encoding, seed: int) -> np.ndarray:
    """Raw GGUF rows [n, row_bytes] whose repeats differ in scale.

    Up to SLAB_ROWS rows are drawn from N(0, 0.02) and quantized.  Taller
    matrices repeat that slab (so a 151936-row LM head stays cheap to build on
    the host) and then give every row its own seeded factors in [0.5, 0.9) or
    [1.1, 1.5) on each fp16 scale field of its blocks (d, and dmin / m where the encoding has
    one).  A kernel that reads row r +- SLAB_ROWS * j, or whose workgroup index
    wraps, then produces output rows off by the ratio of two factors (all but
    the ~0.5% of row pairs whose subnormal Q6_K d rounds to the same fp16)."""
    code = Q.ggml_type(encoding)
    rows = min(n, SLAB_ROWS)
    slab = Q.sample_weight(rows, k, code, seed=seed)
    if rows == n:
        return slab
    reps = -(-n // rows)
    tall = np.ascontiguousarray(np.tile(slab, (reps, 1))[:n])
    rescale_rows(tall, code, np.random.default_rng(seed + 7919))
    return tall


def rescale_rows(raw: np.ndarray, code: int, rng) -> None:
    """Multiply each row's fp16 scale fields, in place, by factors drawn per row and field."""
    qk, size = Q.GEOMETRY[code]
    n = raw.shape[0]
    blocks = raw.reshape(n, -1, size)
    for offset in HALF_FIELDS[code]:
        # at least 10% away from 1, so that the rounded fp16 field changes
        factor = rng.uniform(0.5, 0.9, size=(n, 1)) + 0.6 * rng.integers(0, 2, size=(n, 1))
        factor = factor.astype(np.float32)
        field = np.ascontiguousarray(blocks[:, :, offset:offset + 2]).view(np.float16)[..., 0]
        scaled = (field.astype(np.float32) * factor).astype(np.float16)
        blocks[:, :, offset:offset + 2] = scaled[..., None].view(np.uint8)


def activation(m: int, k: int, seed: int) -> np.ndarray:
    return Q.sample_activation(m, k, seed=seed)


def random_blocks(encoding, n: int, k: int, seed: int, scale: float = 0.05) -> np.ndarray:
    """Random block bytes (every bit pattern of the code fields) with finite fp16 scales."""
    code = Q.ggml_type(encoding)
    qk, size = Q.GEOMETRY[code]
    rng = np.random.default_rng(seed)
    blocks = n * k // qk
    raw = rng.integers(0, 256, size=(blocks, size), dtype=np.uint8)
    for offset in HALF_FIELDS[code]:
        half = (rng.standard_normal(blocks) * scale).astype(np.float16).view(np.uint8).reshape(blocks, 2)
        raw[:, offset:offset + 2] = half
    return raw.reshape(n, -1)


# Byte offsets of each encoding's fp16 fields (d, and m / dmin where present).
HALF_FIELDS = {Q.Q4_0: (0,), Q.Q8_0: (0,), Q.Q4_K: (0, 2), Q.Q6_K: (208,), Q.Q4_1: (0, 2), Q.Q5_0: (0,),
               Q.Q5_1: (0, 2), Q.Q2_K: (80, 82), Q.Q3_K: (108,), Q.Q5_K: (0, 2)}
