"""Host-side GGUF block encoders and seeded weight generation.

The reference takes raw GGML bytes from AKAS ``weight_storage`` /
``sample_weight`` (``benchmarks/kernels/showcase/benchmark.py:453-459``), which
are not vendored.  This module is this package's own producer of the same
bytes: it quantizes fp32 weights into GGML blocks (types 2, 8, 12, 14) whose
layouts are fixed by ``benchmarks/kernels/showcase/triton_kernels.py:134-181``
and the public GGML block definitions, and likewise into types 3, 6, 7, 10, 11
and 13 (Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K: public GGML layouts only).  Quantization happens once, offline, on
the host; it is not on the GPU hot path.

The packers (``pack_*``) place already-chosen integer codes into bytes.  They
are written in the encoder's direction (codes -> bytes) and are what the tests
use to pin every decoder field independently of the decoders themselves.
"""

from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
# The other GGML encodings the kernels decode (public GGML block definitions).
Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K = 3, 6, 7, 10, 11, 13
GEOMETRY = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210),
            Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q2_K: (256, 84), Q3_K: (256, 110),
            Q5_K: (256, 176)}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", Q4_1: "q4_1", Q5_0: "q5_0",
         Q5_1: "q5_1", Q2_K: "q2_k", Q3_K: "q3_k", Q5_K: "q5_k"}
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


def pack_q4_1(d, m, q) -> np.ndarray:
    """d, m: [B]; q: 4-bit codes [B, 32] (value = q * d + m) -> [B, 20]; nibbles as Q4_0."""
    q = np.asarray(q, dtype=np.uint8)
    out = np.empty(np.shape(d) + (20,), dtype=np.uint8)
    out[..., 0:2] = _fp16_bytes(np.asarray(d))
    out[..., 2:4] = _fp16_bytes(np.asarray(m))
    out[..., 4:20] = (q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)
    return out


def _pack_q5(head: list, q) -> np.ndarray:
    """fp16 header fields, then qh (bit j = bit 4 of code j, little-endian u32), then the
    low nibbles as Q4_0 (element j < 16 low nibble of byte j, j + 16 its high nibble)."""
    q = np.asarray(q, dtype=np.uint32)
    count = len(head)
    out = np.empty(q.shape[:-1] + (2 * count + 20,), dtype=np.uint8)
    for i, field in enumerate(head):
        out[..., 2 * i: 2 * i + 2] = _fp16_bytes(np.asarray(field))
    qh = ((q >> 4) & 1) << np.arange(32, dtype=np.uint32)
    out[..., 2 * count: 2 * count + 4] = qh.sum(axis=-1, dtype=np.uint32)[..., None].view(np.uint8)
    low = (q & 15).astype(np.uint8)
    out[..., 2 * count + 4:] = low[..., :16] | (low[..., 16:] << 4)
    return out


def pack_q5_0(d, q) -> np.ndarray:
    """d: [B]; q: 5-bit codes [B, 32] (value = (q - 16) * d) -> [B, 22]."""
    return _pack_q5([d], q)


def pack_q5_1(d, m, q) -> np.ndarray:
    """d, m: [B]; q: 5-bit codes [B, 32] (value = q * d + m) -> [B, 24]."""
    return _pack_q5([d, m], q)


def pack_q2_k(d, dmin, scales, mins, q) -> np.ndarray:
    """Pack a Q2_K super-block.

    d, dmin: [B]; scales, mins: 4-bit codes [B, 16] (one per 16 elements); q: 2-bit
    codes [B, 256].  Value of element e: d*scales[e//16]*q[e] - dmin*mins[e//16].
    Byte s of the 16 scale bytes is scales[s] | mins[s] << 4.  Each 128-element half
    owns 32 code bytes: element h*128 + 32*p + l sits in bits 2p..2p+1 of byte h*32 + l.
    Then fp16 d and fp16 dmin.
    """
    q = np.asarray(q, dtype=np.uint8)
    out = np.zeros(np.shape(d) + (84,), dtype=np.uint8)
    out[..., 0:16] = (np.asarray(scales, dtype=np.uint8) & 15) | ((np.asarray(mins, dtype=np.uint8) & 15) << 4)
    for h in range(2):
        for p in range(4):
            out[..., 16 + 32 * h: 48 + 32 * h] |= (q[..., 128 * h + 32 * p: 128 * h + 32 * p + 32] & 3) << (2 * p)
    out[..., 80:82] = _fp16_bytes(np.asarray(d))
    out[..., 82:84] = _fp16_bytes(np.asarray(dmin))
    return out


def pack_q3_k(d, scales, q) -> np.ndarray:
    """Pack a Q3_K super-block.

    d: [B]; scales: signed 6-bit [B, 16] in -32..31 (one per 16 elements); q: signed
    3-bit codes [B, 256] in -4..3.  Value of element e: d * scales[e//16] * q[e].
    Code c = q + 4: its low 2 bits sit like Q2_K's codes (32 bytes after the 32-byte
    mask), its bit 2 in mask byte e % 32 at bit (e // 128) * 4 + (e % 128) // 32.
    Scale s is stored as u = scales[s] + 32: the low nibble in byte s (s < 8) or the
    high nibble of byte s - 8 (s >= 8) of the 12 scale bytes, the top 2 bits in byte
    8 + s % 4 at bit 2 * (s // 4).  Then fp16 d.
    """
    code = (np.asarray(q, dtype=np.int16) + 4).astype(np.uint8)
    u = (np.asarray(scales, dtype=np.int16) + 32).astype(np.uint8)
    out = np.zeros(np.shape(d) + (110,), dtype=np.uint8)
    for e0 in range(0, 256, 32):
        h, p = e0 // 128, e0 % 128 // 32
        part = code[..., e0: e0 + 32]
        out[..., 0:32] |= ((part >> 2) & 1) << (4 * h + p)
        out[..., 32 + 32 * h: 64 + 32 * h] |= (part & 3) << (2 * p)
    for index in range(16):
        low, high = u[..., index] & 15, (u[..., index] >> 4) & 3
        out[..., 96 + index % 8] |= low << (4 * (index // 8))
        out[..., 104 + index % 4] |= high << (2 * (index // 4))
    out[..., 108:110] = _fp16_bytes(np.asarray(d))
    return out


def pack_q5_k(d, dmin, scales, mins, q) -> np.ndarray:
    """Pack a Q5_K super-block: Q4_K's header and nibble layout for the low 4 bits of
    the 5-bit codes q [B, 256], with bit 4 of element e in byte e % 32 of the 32-byte
    qh run at bit e // 32.  Value: d*scales[e//32]*q[e] - dmin*mins[e//32]."""
    q = np.asarray(q, dtype=np.uint8)
    q4k = pack_q4_k(d, dmin, scales, mins, q & 15)
    out = np.zeros(np.shape(d) + (176,), dtype=np.uint8)
    out[..., 0:16] = q4k[..., 0:16]
    for sub in range(8):
        out[..., 16:48] |= ((q[..., 32 * sub: 32 * sub + 32] >> 4) & 1) << sub
    out[..., 48:176] = q4k[..., 16:144]
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


def _affine_codes(blocks, levels):
    """Per-block affine fit [lo, hi] -> (step, lo, codes 0..levels) with round-half-away."""
    lo, hi = blocks.min(axis=-1), blocks.max(axis=-1)
    step = ((hi - lo) / levels).astype(np.float16).astype(np.float32)
    base = lo.astype(np.float16).astype(np.float32)
    safe = np.where(step > 0, step, 1.0)
    codes = np.where(step[..., None] > 0, _round_half_away((blocks - base[..., None]) / safe[..., None]), 0)
    return step, base, np.clip(codes, 0, levels).astype(np.uint8)


def quantize_q4_1(w: np.ndarray) -> np.ndarray:
    """Q4_1: per 32 values d = (max - min)/15 and m = min, q = round((x - m)/d)."""
    step, base, q = _affine_codes(np.asarray(w, dtype=np.float32).reshape(-1, 32), 15)
    return pack_q4_1(step, base, q)


def quantize_q5_1(w: np.ndarray) -> np.ndarray:
    """Q5_1: per 32 values d = (max - min)/31 and m = min."""
    step, base, q = _affine_codes(np.asarray(w, dtype=np.float32).reshape(-1, 32), 31)
    return pack_q5_1(step, base, q)


def quantize_q5_0(w: np.ndarray) -> np.ndarray:
    """Q5_0: the signed extreme maps to code 0 (d = extreme / -16), as Q4_0 does with -8."""
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    extreme = blocks[np.arange(blocks.shape[0]), np.abs(blocks).argmax(axis=1)]
    d = (extreme / -16.0).astype(np.float16).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.floor(blocks * inv[:, None] + 16.5), 0, 31).astype(np.uint8)
    return pack_q5_0(d, q)


def _k_affine(blocks, levels, scale_levels):
    """K-quant affine fit: per sub-block step (hi - lo)/levels and offset -lo (lo <= 0),
    both quantized against the super-block's d and dmin (largest / scale_levels)."""
    lo = np.minimum(blocks.min(axis=2), 0.0)
    step = (blocks.max(axis=2) - lo) / levels
    offset = -lo
    d = (step.max(axis=1) / scale_levels).astype(np.float16)
    dmin = (offset.max(axis=1) / scale_levels).astype(np.float16)
    d32, dmin32 = d.astype(np.float32), dmin.astype(np.float32)
    scales = np.clip(_round_half_away(step / np.where(d32 > 0, d32, 1.0)[:, None]), 0, scale_levels)
    mins = np.clip(_round_half_away(offset / np.where(dmin32 > 0, dmin32, 1.0)[:, None]), 0, scale_levels)
    unit = d32[:, None] * scales.astype(np.float32)
    base = dmin32[:, None] * mins.astype(np.float32)
    q = _round_half_away((blocks + base[:, :, None]) / np.where(unit > 0, unit, 1.0)[:, :, None])
    q = np.where(unit[:, :, None] > 0, np.clip(q, 0, levels), 0).astype(np.uint8)
    return d, dmin, scales.astype(np.uint8), mins.astype(np.uint8), q.reshape(blocks.shape[0], -1)


def quantize_q2_k(w: np.ndarray) -> np.ndarray:
    """Q2_K: 2-bit codes with a 4-bit (step, offset) pair per 16 elements."""
    return pack_q2_k(*_k_affine(np.asarray(w, dtype=np.float32).reshape(-1, 16, 16), 3, 15))


def quantize_q5_k(w: np.ndarray) -> np.ndarray:
    """Q5_K: 5-bit codes with 6-bit (step, offset) pairs per 32 elements."""
    return pack_q5_k(*_k_affine(np.asarray(w, dtype=np.float32).reshape(-1, 8, 32), 31, 63))


def quantize_q3_k(w: np.ndarray) -> np.ndarray:
    """Q3_K: per 16 elements the signed extreme maps to code -4; the sixteen signed
    6-bit scales are quantized against d = largest / -32."""
    blocks = np.asarray(w, dtype=np.float32).reshape(-1, 16, 16)
    extreme = np.take_along_axis(blocks, np.abs(blocks).argmax(axis=2)[:, :, None], axis=2)[:, :, 0]
    sub = extreme / -4.0
    big = np.take_along_axis(sub, np.abs(sub).argmax(axis=1)[:, None], axis=1)[:, 0]
    d = (big / -32.0).astype(np.float16).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    scales = np.clip(_round_half_away(sub * inv[:, None]), -32, 31)
    unit = d[:, None] * scales.astype(np.float32)
    q = _round_half_away(blocks / np.where(unit != 0, unit, 1.0)[:, :, None])
    q = np.where(unit[:, :, None] != 0, np.clip(q, -4, 3), 0)
    return pack_q3_k(d, scales.astype(np.int8), q.astype(np.int8).reshape(-1, 256))


QUANTIZERS = {Q4_0: quantize_q4_0, Q8_0: quantize_q8_0, Q4_K: quantize_q4_k, Q6_K: quantize_q6_k,
              Q4_1: quantize_q4_1, Q5_0: quantize_q5_0, Q5_1: quantize_q5_1, Q2_K: quantize_q2_k,
              Q3_K: quantize_q3_k, Q5_K: quantize_q5_k}


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
