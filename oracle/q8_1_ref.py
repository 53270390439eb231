"""ORACLE -- test infrastructure only (the same rules as ``gguf_ref``: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it).

CPU restatement of the Q8_1-activation integer-dot decode GEMV, GGML's path for quantized
matrix-vector products, which the reference measures as its external GGML baseline
(``benchmarks/kernels/showcase/external_baselines.py:24-58``: "GGML may quantize F32
activations to Q8_1", qualified at relative L2 <= 0.02 against the fp32 oracle).  GGML itself is
not part of the reference tree (the showcase builds a bridge against a separate llama.cpp
checkout, ``benchmarks/kernels/showcase/README.md:57-73``, no version pinned), so this module
restates the published algorithm of ggml's ``block_q8_1`` and its dot products:

* activations in blocks of 32: ``d = max|x| / 127``, ``q = roundf(x / d)`` (half away from
  zero, computed as ``x * (1 / d)``, 0 for an all-zero block), the block stores ``d`` and
  ``s = d * sum(q)``, both as fp16 (ggml's ``quantize_row_q8_1``);
* a weight block meets one or two activation blocks through integer dot products of the codes,
  and the per-block scales are applied in fp32:

  - Q8_0:  ``(d_w * d_x) * sum(q_w q_x)``
  - Q4_0:  ``d_w * (d_x * sum(q_w q_x) - 8 s_x)`` with ``q_w`` in 0..15 (the -8 offset folded
    into the block sum)
  - Q4_K:  per 32-element sub-block ``j``: ``(d sc_j) * (d_x * sum(q q_x)) - (dmin m_j) * s_x``
  - Q6_K:  per 32-element run, two 16-element scale groups:
    ``(d * d_x) * (sc_0 sum_0((q - 32) q_x) + sc_1 sum_1((q - 32) q_x))``

  every integer sum is exact (at most 2^24 in magnitude), and the contributions of the
  ``K / 32`` activation blocks are added in block order in fp32.

Pinned by ``tests/test_q8_1_oracle.py``: the quantizer against its defining properties (round
trip within d / 2, the largest element at +-127, ties away from zero, zero blocks) and the dot
products against an fp64 sum of the decoded weights (``gguf_ref.dequantize``) times the decoded
activations (``d * q``), which a dropped min term, a wrong offset or a misplaced scale fails.
"""

from __future__ import annotations

import numpy as np

from oracle import gguf_ref as R

Q8_1_BLOCK = 32
TYPES = (R.Q4_0, R.Q8_0, R.Q4_K, R.Q6_K)


def _fp16(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).astype(np.float32)


def quantize_q8_1(x: np.ndarray):
    """(q int8 [M, K], d fp32 [M, K/32], s fp32 [M, K/32]) of fp32 activations [M, K];
    d and s hold their fp16 values."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    if k % Q8_1_BLOCK:
        raise ValueError("K must be a multiple of 32")
    blocks = x.reshape(m, k // Q8_1_BLOCK, Q8_1_BLOCK)
    amax = np.abs(blocks).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (blocks * inv[:, :, None]).astype(np.float32).astype(np.float64)  # exact widening
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int32)        # roundf: half away from zero
    s = (np.float32(1.0) * q.sum(axis=2).astype(np.float32) * d).astype(np.float32)
    return q.reshape(m, k).astype(np.int8), _fp16(d), _fp16(s)


def _weight_blocks(raw: np.ndarray, ggml_type: int, n: int, k: int):
    """Per 32-element block of W: the integer codes (int8 [n, k/32, 32]) as the dot product
    takes them, and the block's scale fields."""
    qk, size = R.GEOMETRY[ggml_type]
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(n, k // qk * size)
    nb = k // Q8_1_BLOCK

    def half(lo, hi):
        return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float32)

    if ggml_type in (R.Q4_0, R.Q8_0):
        blocks = raw.reshape(n, nb, size)
        d = half(blocks[:, :, 0], blocks[:, :, 1])
        if ggml_type == R.Q8_0:
            codes = blocks[:, :, 2:].view(np.int8)
        else:  # byte i: element i (low nibble), element i + 16 (high nibble)
            quants = blocks[:, :, 2:]
            codes = np.concatenate([quants & 15, quants >> 4], axis=2).astype(np.int8)
        return codes, {"d": d}
    supers = raw.reshape(n, k // 256, size)
    if ggml_type == R.Q4_K:
        d, dmin = half(supers[:, :, 0], supers[:, :, 1]), half(supers[:, :, 2], supers[:, :, 3])
        s0, s1, s2 = (supers[:, :, o:o + 4].astype(np.int32) for o in (4, 8, 12))
        sc = np.concatenate([s0 & 63, (s2 & 15) | ((s0 >> 6) << 4)], axis=2)   # sub-blocks 0..7
        mn = np.concatenate([s1 & 63, (s2 >> 4) | ((s1 >> 6) << 4)], axis=2)
        # quant pair p (bytes 16 + 32 p + l): low nibbles are sub-block 2p, high nibbles 2p + 1
        quants = supers[:, :, 16:144].reshape(n, -1, 4, 1, 32)
        codes = np.concatenate([quants & 15, quants >> 4], axis=3).astype(np.int8).reshape(n, nb, 32)
        return codes, {"d": np.repeat(d, 8, axis=1), "dmin": np.repeat(dmin, 8, axis=1),
                       "sc": sc.reshape(n, nb), "m": mn.reshape(n, nb)}
    # Q6_K: block j = 4 h + c holds elements 128 h + 32 c + l: low bits from byte
    # 64 h + 32 (c % 2) + l (nibble c / 2), high bits from byte 128 + 32 h + l (bits 2c, 2c + 1)
    ql = supers[:, :, 0:128].reshape(n, -1, 2, 2, 32)
    qh = supers[:, :, 128:192].reshape(n, -1, 2, 32)
    runs = [((ql[:, :, :, c % 2] >> (4 * (c // 2))) & 15) | (((qh >> (2 * c)) & 3) << 4) for c in range(4)]
    q = np.stack(runs, axis=3).astype(np.int16) - 32                     # [n, S, h, c, 32]
    scales = supers[:, :, 192:208].view(np.int8).astype(np.int32).reshape(n, nb, 2)  # scales 2j, 2j + 1
    d = half(supers[:, :, 208], supers[:, :, 209])
    return q.astype(np.int8).reshape(n, nb, 32), {"d": np.repeat(d, 8, axis=1), "sc": scales}


def gemv_q8_1(x: np.ndarray, raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
    """out [M, N] (fp32) of the Q8_1 integer-dot GEMV: x quantized to Q8_1, one fp32
    contribution per 32-element block, added in block order."""
    if ggml_type not in TYPES:
        raise ValueError(f"no Q8_1 dot product for GGML type {ggml_type}")
    x = np.asarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    q, dx, sx = quantize_q8_1(x)
    nb = k // Q8_1_BLOCK
    # integer sums of every (row, block) pair, by block: every partial sum of at most 32 products
    # of the codes stays below 2^24 in magnitude, so fp32 matrix products give them exactly
    qb = np.ascontiguousarray(q.reshape(m, nb, 32).transpose(1, 2, 0).astype(np.float32))  # [nb, 32, m]
    codes, f = _weight_blocks(raw, ggml_type, n, k)
    wb = np.ascontiguousarray(codes.transpose(1, 0, 2).astype(np.float32))                 # [nb, n, 32]
    if ggml_type == R.Q6_K:
        g0 = np.matmul(wb[:, :, :16], qb[:, :16, :])  # [nb, n, m]: the two 16-element scale groups
        g1 = np.matmul(wb[:, :, 16:], qb[:, 16:, :])
        sc = f["sc"].astype(np.float32)                                                 # [n, nb, 2]
        isums = g0 * sc.transpose(1, 0, 2)[:, :, 0:1] + g1 * sc.transpose(1, 0, 2)[:, :, 1:2]
    else:
        isums = np.matmul(wb, qb)                                                      # [nb, n, m]
    isums = isums.transpose(0, 2, 1).astype(np.float32)                                # [nb, m, n], exact
    acc = np.zeros((m, n), dtype=np.float32)
    for b in range(nb):
        isum = isums[b]
        if ggml_type in (R.Q6_K, R.Q8_0):
            c = (f["d"][None, :, b] * dx[:, None, b]).astype(np.float32) * isum
        elif ggml_type == R.Q4_0:
            c = f["d"][None, :, b] * ((dx[:, None, b] * isum).astype(np.float32)
                                      - np.float32(8.0) * sx[:, None, b]).astype(np.float32)
        else:
            scale = (f["d"][:, b] * f["sc"][:, b].astype(np.float32)).astype(np.float32)
            offset = (f["dmin"][:, b] * f["m"][:, b].astype(np.float32)).astype(np.float32)
            c = (scale[None, :] * (dx[:, None, b] * isum).astype(np.float32)).astype(np.float32) \
                - (offset[None, :] * sx[:, None, b]).astype(np.float32)
        acc = (acc + c.astype(np.float32)).astype(np.float32)
    return acc


def gemv_q8_1_exact(x: np.ndarray, raw: np.ndarray, ggml_type: int, n: int, k: int) -> np.ndarray:
    """The same product in fp64 from the decoded operands: dequant(W) (``gguf_ref.dequantize``)
    times d * q of the Q8_1 activations.  For Q4_0 and Q4_K the fp16 block sum ``s`` stands in for
    d * sum(q) in the offset and min terms, as the integer-dot form uses it."""
    x = np.asarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    q, dx, sx = quantize_q8_1(x)
    xq = (q.reshape(m, k // 32, 32).astype(np.float64) * dx[:, :, None].astype(np.float64)).reshape(m, k)
    w = R.dequantize(raw, ggml_type, n, k).astype(np.float64)
    out = xq @ w.T
    if ggml_type in (R.Q4_0, R.Q4_K):
        # replace d * sum(q) by its fp16 value s in the terms that multiply a block-constant part
        # of W: -8 d_w (Q4_0) and -dmin m_j (Q4_K)
        codes, f = _weight_blocks(raw, ggml_type, n, k)
        if ggml_type == R.Q4_0:
            const = -8.0 * f["d"].astype(np.float64)                              # [n, k/32]
        else:
            const = -(f["dmin"].astype(np.float64) * f["m"].astype(np.float64))
        exact_sum = (q.reshape(m, k // 32, 32).astype(np.float64).sum(axis=2) * dx.astype(np.float64))
        out += (sx.astype(np.float64) - exact_sum) @ const.T
    return out
