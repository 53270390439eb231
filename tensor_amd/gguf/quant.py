"""Host-side GGUF block encoders and seeded weight generation.

The reference takes raw GGML bytes from AKAS ``weight_storage`` /
``sample_weight`` (``benchmarks/kernels/showcase/benchmark.py:453-459``), which
are not vendored.  This module is this package's own producer of the same
bytes: it quantizes fp32 weights into GGML blocks (types 2, 8, 12, 14) whose
layouts are fixed by ``benchmarks/kernels/showcase/triton_kernels.py:134-181``
and the public GGML block definitions.  Quantization happens once, offline, on
the host; it is not on the GPU hot path.

The packers (``pack_*``) place already-chosen integer codes into bytes.  They
are written in the encoder's direction (codes -> bytes) and are what the tests
use to pin every decoder field independently of the decoders themselves.
"""

from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
GEOMETRY = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}
TYPES = {name: code for code, name in NAMES.items()}


def ggml_type(value) -> int:
    """Accept a GGML type id or its name ("q4_k", "Q6_K", ...)."""
    if isinstance(value, str):
        try:
            return TYPES[value.lower()]
        except KeyError:
            raise ValueError(f"unsupported GGUF encoding {value!r}") from None
    if int(value) not in GEOMETRY:
        raise ValueError(f"unsupported GGML type {value!r}")
    return int(value)


def row_bytes(ggml: int, k: int) -> int:
    qk, block = GEOMETRY[ggml]
    if k % qk:
        raise ValueError(f"K={k} is not a multiple of the {NAMES[ggml]} block size {qk}")
    return k // qk * block


def _fp16_bytes(values: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(values.astype(np.float16)).view(np.uint8).reshape(values.shape + (2,))


def _round_half_away(values: np.ndarray) -> np.ndarray:
    """C roundf(): halves round away from zero (numpy rounds them to even)."""
    return np.sign(values) * np.floor(np.abs(values) + 0.5)


# ------------------------------------------------------------------ packers --

def pack_q8_0(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """d: fp16-able [B]; q: int8 codes [B, 32] -> [B, 34] bytes."""
    out = np.empty(d.shape + (34,), dtype=np.uint8)
    out[..., 0:2] = _fp16_bytes(d)
    out[..., 2:34] = q.astype(np.int8).view(np.uint8)
    return out


def pack_q4_0(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """d: [B]; q: unsigned 4-bit codes [B, 32] (value = (q - 8) * d) -> [B, 18].

    Element j < 16 is the low nibble of byte j, element j + 16 its high nibble.
    """
    q = q.astype(np.uint8)
    out = np.empty(d.shape + (18,), dtype=np.uint8)
    out[..., 0:2] = _fp16_bytes(d)
    out[..., 2:18] = q[..., :16] | (q[..., 16:] << 4)
    return out


def pack_q4_k(d, dmin, scales, mins, q) -> np.ndarray:
    """Pack a Q4_K super-block.

    d, dmin: [B]; scales, mins: 6-bit codes [B, 8]; q: 4-bit codes [B, 256].
    Value of element e in sub-block s = e // 32:  d*scales[s]*q[e] - dmin*mins[s].

    Scale bytes: sub-blocks 0-3 keep their 6-bit scale in byte s and 6-bit min
    in byte s + 4; sub-blocks 4-7 keep the low 4 bits of scale and min in byte
    s + 4 (scale low nibble, min high nibble) and spill their top 2 bits into
    the spare top bits of bytes s - 4 (scale) and s (min).
    Quants: each 64-element group owns 32 bytes; element g*64 + l sits in the
    low nibble of byte g*32 + l, element g*64 + 32 + l in its high nibble.
    """
    scales = np.asarray(scales, dtype=np.uint8)
    mins = np.asarray(mins, dtype=np.uint8)
    q = np.asarray(q, dtype=np.uint8)
    out = np.zeros(np.shape(d) + (144,), dtype=np.uint8)
    out[..., 0:2] = _fp16_bytes(np.asarray(d))
    out[..., 2:4] = _fp16_bytes(np.asarray(dmin))
    packed = np.zeros(np.shape(d) + (12,), dtype=np.uint8)
    for s in range(8):
        sc, mn = scales[..., s], mins[..., s]
        if s < 4:
            packed[..., s] |= sc & 63
            packed[..., s + 4] |= mn & 63
        else:
            packed[..., s + 4] |= (sc & 15) | ((mn & 15) << 4)
            packed[..., s - 4] |= (sc >> 4) << 6
            packed[..., s] |= (mn >> 4) << 6
    out[..., 4:16] = packed
    for g in range(4):
        low = q[..., 64 * g: 64 * g + 32]
        high = q[..., 64 * g + 32: 64 * g + 64]
        out[..., 16 + 32 * g: 16 + 32 * g + 32] = (low & 15) | ((high & 15) << 4)
    return out


def pack_q6_k(d, scales, q) -> np.ndarray:
    """Pack a Q6_K super-block.

    d: [B]; scales: int8 [B, 16] (one per 16 elements); q: 6-bit codes [B, 256]
    (value = d * scales[e // 16] * (q[e] - 32)).
    Each 128-element half owns 64 low-nibble bytes and 32 high-bit bytes:
    for l < 32 the four elements h*128 + l + 32*c (c = 0..3) put their low
    nibbles in ql[h*64 + l] (c = 0 low, c = 2 high) and ql[h*64 + 32 + l]
    (c = 1 low, c = 3 high), and their top 2 bits in qh[h*32 + l] at bit 2*c.
    """
    q = np.asarray(q, dtype=np.uint8)
    out = np.zeros(np.shape(d) + (210,), dtype=np.uint8)
    for h in range(2):
        part = [q[..., 128 * h + 32 * c: 128 * h + 32 * c + 32] for c in range(4)]
        out[..., 64 * h: 64 * h + 32] = (part[0] & 15) | ((part[2] & 15) << 4)
        out[..., 64 * h + 32: 64 * h + 64] = (part[1] & 15) | ((part[3] & 15) << 4)
        out[..., 128 + 32 * h: 128 + 32 * h + 32] = (
            (part[0] >> 4) | ((part[1] >> 4) << 2) | ((part[2] >> 4) << 4) | ((part[3] >> 4) << 6)
        )
    out[..., 192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    out[..., 208:210] = _fp16_bytes(np.asarray(d))
    return out


# ---------------------------------------------------------------- quantizers --

def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """GGML-style Q8_0: d = absmax/127 per 32 values, q = round(x/d)."""
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    d = amax / 127.0
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(_round_half_away(blocks * inv[:, None]), -127, 127).astype(np.int8)
    return pack_q8_0(d.astype(np.float32), q)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """GGML-style Q4_0: the signed extreme maps to code 0 (d = extreme / -8)."""
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    index = np.abs(blocks).argmax(axis=1)
    extreme = blocks[np.arange(blocks.shape[0]), index]
    d = (extreme / -8.0).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.floor(blocks * inv[:, None] + 8.5), 0, 15).astype(np.uint8)
    return pack_q4_0(d, q)


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """Q4_K with an affine fit per 32-element sub-block.

    Each sub-block spans [lo, hi] with lo <= 0; its step (hi - lo)/15 and its
    offset -lo are quantized to 6 bits against the super-block's d and dmin
    (each the largest of the eight divided by 63), then every element takes
    the nearest 4-bit code under the quantized step and offset.
    """
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 8, 32)
    lo = np.minimum(blocks.min(axis=2), 0.0)
    hi = blocks.max(axis=2)
    step = (hi - lo) / 15.0
    offset = -lo
    d = (step.max(axis=1) / 63.0).astype(np.float16)
    dmin = (offset.max(axis=1) / 63.0).astype(np.float16)
    d32, dmin32 = d.astype(np.float32), dmin.astype(np.float32)
    safe_d = np.where(d32 > 0, d32, 1.0)
    safe_m = np.where(dmin32 > 0, dmin32, 1.0)
    scales = np.clip(_round_half_away(step / safe_d[:, None]), 0, 63).astype(np.uint8)
    mins = np.clip(_round_half_away(offset / safe_m[:, None]), 0, 63).astype(np.uint8)
    unit = d32[:, None] * scales.astype(np.float32)
    base = dmin32[:, None] * mins.astype(np.float32)
    safe_unit = np.where(unit > 0, unit, 1.0)
    q = _round_half_away((blocks + base[:, :, None]) / safe_unit[:, :, None])
    q = np.where(unit[:, :, None] > 0, np.clip(q, 0, 15), 0).astype(np.uint8)
    return pack_q4_k(d, dmin, scales, mins, q.reshape(-1, 256))


def quantize_q6_k(w: np.ndarray) -> np.ndarray:
    """Q6_K: per 16 elements the signed extreme maps to code -32; the sixteen
    sub-block scales are quantized to int8 against d = largest / -128."""
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 16, 16)
    index = np.abs(blocks).argmax(axis=2)
    extreme = np.take_along_axis(blocks, index[:, :, None], axis=2)[:, :, 0]
    sub = extreme / -32.0
    big = np.take_along_axis(sub, np.abs(sub).argmax(axis=1)[:, None], axis=1)[:, 0]
    inv = np.where(big != 0, -128.0 / np.where(big != 0, big, 1.0), 0.0).astype(np.float32)
    scales = np.clip(_round_half_away(sub * inv[:, None]), -128, 127).astype(np.int8)
    d = np.where(inv != 0, 1.0 / np.where(inv != 0, inv, 1.0), 0.0).astype(np.float16)
    unit = d.astype(np.float32)[:, None] * scales.astype(np.float32)
    safe = np.where(unit != 0, unit, 1.0)
    q = _round_half_away(blocks / safe[:, :, None])
    q = np.where(unit[:, :, None] != 0, np.clip(q, -32, 31), 0) + 32
    return pack_q6_k(d, scales, q.astype(np.uint8).reshape(-1, 256))


QUANTIZERS = {Q4_0: quantize_q4_0, Q8_0: quantize_q8_0, Q4_K: quantize_q4_k, Q6_K: quantize_q6_k}


def quantize(w: np.ndarray, encoding) -> np.ndarray:
    """Quantize an [N, K] fp32 matrix into raw rows of shape [N, row_bytes]."""
    code = ggml_type(encoding)
    w = np.asarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("weight must be a 2-D [N, K] matrix")
    n, k = w.shape
    return QUANTIZERS[code](w).reshape(n, row_bytes(code, k))


def sample_weight(n: int, k: int, encoding, *, seed: int, std: float = 0.02,
                  chunk_rows: int = 4096) -> np.ndarray:
    """Seeded N(0, std) weights (numpy PCG64) quantized to raw GGML rows.

    Rows are generated and quantized in chunks so a 151936 x 4096 LM head
    never needs its fp32 matrix in memory at once.  The stream is identical
    to drawing the whole [N, K] matrix at once.
    """
    code = ggml_type(encoding)
    rng = np.random.Generator(np.random.PCG64(seed))
    out = np.empty((n, row_bytes(code, k)), dtype=np.uint8)
    for start in range(0, n, chunk_rows):
        rows = min(chunk_rows, n - start)
        block = rng.standard_normal((rows, k), dtype=np.float32) * np.float32(std)
        out[start:start + rows] = QUANTIZERS[code](block).reshape(rows, -1)
    return out


def sample_activation(m: int, k: int, *, seed: int) -> np.ndarray:
    """Seeded N(0, 1) activations stored as fp16 [M, K]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
