"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

The reference holds no GGUF golden vectors (no test touches GGUF), so every
decoder field is pinned here by construction: blocks are built with the
encoder-direction packers of ``tensor_amd.gguf.quant`` from chosen integer
codes, under scales that make the decoded value a closed form of those codes
(d = 1, dmin = 0, unit scales ...), and both independent oracles (NumPy per-
element formulas and the C block walker) must reproduce it exactly.  A wrong
shift, a swapped byte index or a misplaced field fails one of these.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q

TYPES = (Q.Q4_0, Q.Q8_0, Q.Q4_K, Q.Q6_K)
# Encodings restated from the public GGML block definitions only.
MORE = (Q.Q4_1, Q.Q5_0, Q.Q5_1, Q.Q2_K, Q.Q3_K, Q.Q5_K)


def both(raw, t, n, k, c_oracle):
    a = R.dequantize(raw, t, n, k)
    b = c_oracle.dequantize(raw, t, n, k)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "numpy and C oracles disagree"
    return a


# Byte offsets of each encoding's fp16 fields.
HALF_FIELDS = {Q.Q4_0: (0,), Q.Q8_0: (0,), Q.Q4_K: (0, 2), Q.Q6_K: (208,), Q.Q4_1: (0, 2), Q.Q5_0: (0,),
               Q.Q5_1: (0, 2), Q.Q2_K: (80, 82), Q.Q3_K: (108,), Q.Q5_K: (0, 2)}


def random_blocks(t, blocks, rng):
    """Random bytes with every fp16 scale field replaced by a finite value."""
    qk, size = Q.GEOMETRY[t]
    raw = rng.integers(0, 256, size=(blocks, size), dtype=np.uint8)
    for offset in HALF_FIELDS[t]:
        half = (rng.standard_normal(blocks) * 0.05).astype(np.float16).view(np.uint8).reshape(blocks, 2)
        raw[:, offset:offset + 2] = half
    return raw


@pytest.mark.parametrize("t", TYPES + MORE)
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_numpy_and_c_decoders_agree_bitwise(t, seed, c_oracle):
    rng = np.random.default_rng(seed)
    qk, size = Q.GEOMETRY[t]
    n, k = 16, 4 * 256
    raw = random_blocks(t, n * k // qk, rng)
    both(raw, t, n, k, c_oracle)


def test_q4k_scale_min_packing_exhaustive(c_oracle):
    """All 64 x 64 (scale, min) pairs in each of the 8 sub-block positions."""
    sc, mn = np.meshgrid(np.arange(64), np.arange(64), indexing="ij")
    sc, mn = sc.reshape(-1), mn.reshape(-1)
    rng = np.random.default_rng(7)
    for sub in range(8):
        blocks = sc.size
        scales = rng.integers(0, 64, size=(blocks, 8))
        mins = rng.integers(0, 64, size=(blocks, 8))
        scales[:, sub], mins[:, sub] = sc, mn
        q = np.ones((blocks, 256), dtype=np.uint8)
        raw = Q.pack_q4_k(np.ones(blocks), np.ones(blocks), scales, mins, q)
        got = both(raw, Q.Q4_K, blocks, 256, c_oracle)
        # d = dmin = 1, q = 1: element e of sub-block s decodes to scales[s] - mins[s]
        expected = np.repeat((scales - mins).astype(np.float32), 32, axis=1)
        assert np.array_equal(got, expected), f"sub-block {sub}"


def test_q4k_nibble_layout(c_oracle):
    rng = np.random.default_rng(3)
    blocks = 64
    q = rng.integers(0, 16, size=(blocks, 256), dtype=np.uint8)
    raw = Q.pack_q4_k(np.ones(blocks), np.zeros(blocks), np.ones((blocks, 8)), np.zeros((blocks, 8)), q)
    got = both(raw, Q.Q4_K, blocks, 256, c_oracle)
    assert np.array_equal(got, q.astype(np.float32))


def test_q4k_d_and_dmin_fields(c_oracle):
    rng = np.random.default_rng(4)
    blocks = 256
    d = rng.standard_normal(blocks).astype(np.float16)
    dmin = rng.standard_normal(blocks).astype(np.float16)
    scales = rng.integers(0, 64, size=(blocks, 8))
    mins = rng.integers(0, 64, size=(blocks, 8))
    q = rng.integers(0, 16, size=(blocks, 256), dtype=np.uint8)
    raw = Q.pack_q4_k(d, dmin, scales, mins, q)
    got = both(raw, Q.Q4_K, blocks, 256, c_oracle)
    # exact products; the subtraction is computed in fp64 and rounded once
    ds = d.astype(np.float64)[:, None] * np.repeat(scales, 32, axis=1)
    dm = dmin.astype(np.float64)[:, None] * np.repeat(mins, 32, axis=1)
    expected = (ds * q - dm).astype(np.float32)
    assert np.array_equal(got, expected)


def test_q6k_code_layout(c_oracle):
    rng = np.random.default_rng(5)
    blocks = 64
    q = rng.integers(0, 64, size=(blocks, 256), dtype=np.uint8)
    raw = Q.pack_q6_k(np.ones(blocks), np.ones((blocks, 16), dtype=np.int8), q)
    got = both(raw, Q.Q6_K, blocks, 256, c_oracle)
    assert np.array_equal(got, q.astype(np.float32) - 32)
    # every one of the 64 codes occurs
    assert len(np.unique(q)) == 64


def test_q6k_scale_and_d_fields(c_oracle):
    rng = np.random.default_rng(6)
    blocks = 128
    d = rng.standard_normal(blocks).astype(np.float16)
    scales = rng.integers(-128, 128, size=(blocks, 16)).astype(np.int8)
    q = rng.integers(0, 64, size=(blocks, 256), dtype=np.uint8)
    raw = Q.pack_q6_k(d, scales, q)
    got = both(raw, Q.Q6_K, blocks, 256, c_oracle)
    expected = (d.astype(np.float64)[:, None] * np.repeat(scales.astype(np.float64), 16, axis=1)
                * (q.astype(np.float64) - 32)).astype(np.float32)
    assert np.array_equal(got, expected)


def test_q8_0_layout(c_oracle):
    rng = np.random.default_rng(8)
    blocks = 256
    d = rng.standard_normal(blocks).astype(np.float16)
    q = rng.integers(-128, 128, size=(blocks, 32)).astype(np.int8)
    raw = Q.pack_q8_0(d, q)
    got = both(raw, Q.Q8_0, blocks, 32, c_oracle)
    assert np.array_equal(got, (d.astype(np.float64)[:, None] * q).astype(np.float32))


def test_q4_0_layout(c_oracle):
    rng = np.random.default_rng(9)
    blocks = 256
    d = rng.standard_normal(blocks).astype(np.float16)
    q = rng.integers(0, 16, size=(blocks, 32), dtype=np.uint8)
    raw = Q.pack_q4_0(d, q)
    got = both(raw, Q.Q4_0, blocks, 32, c_oracle)
    assert np.array_equal(got, (d.astype(np.float64)[:, None] * (q.astype(np.float64) - 8)).astype(np.float32))


def fp16(rng, shape):
    return rng.standard_normal(shape).astype(np.float16)


def test_q4_1_layout(c_oracle):
    rng = np.random.default_rng(11)
    blocks = 256
    d, m = fp16(rng, blocks), fp16(rng, blocks)
    q = rng.integers(0, 16, size=(blocks, 32), dtype=np.uint8)
    got = both(Q.pack_q4_1(d, m, q), Q.Q4_1, blocks, 32, c_oracle)
    # q*d is exact; the addition rounds once
    expected = (d.astype(np.float64)[:, None] * q + m.astype(np.float64)[:, None]).astype(np.float32)
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("t", [Q.Q5_0, Q.Q5_1])
def test_q5_high_bit_and_nibble_layout(t, c_oracle):
    rng = np.random.default_rng(12)
    blocks = 256
    d, m = fp16(rng, blocks), fp16(rng, blocks)
    q = rng.integers(0, 32, size=(blocks, 32), dtype=np.uint8)
    q[0] = np.arange(32)  # every code, every position of the high-bit word
    q[1] = 31 - np.arange(32)
    if t == Q.Q5_0:
        got = both(Q.pack_q5_0(d, q), t, blocks, 32, c_oracle)
        expected = d.astype(np.float64)[:, None] * (q.astype(np.float64) - 16)
    else:
        got = both(Q.pack_q5_1(d, m, q), t, blocks, 32, c_oracle)
        expected = d.astype(np.float64)[:, None] * q + m.astype(np.float64)[:, None]
    assert np.array_equal(got, expected.astype(np.float32))
    # the unit-scale block decodes to the codes themselves
    unit = both(Q.pack_q5_1(np.ones(1), np.zeros(1), q[:1]), Q.Q5_1, 1, 32, c_oracle)
    assert np.array_equal(unit[0], np.arange(32, dtype=np.float32))


def test_q2_k_fields(c_oracle):
    rng = np.random.default_rng(13)
    blocks = 256
    d, dmin = fp16(rng, blocks), fp16(rng, blocks)
    scales = rng.integers(0, 16, size=(blocks, 16))
    mins = rng.integers(0, 16, size=(blocks, 16))
    q = rng.integers(0, 4, size=(blocks, 256), dtype=np.uint8)
    got = both(Q.pack_q2_k(d, dmin, scales, mins, q), Q.Q2_K, blocks, 256, c_oracle)
    ds = d.astype(np.float64)[:, None] * np.repeat(scales, 16, axis=1)
    dm = dmin.astype(np.float64)[:, None] * np.repeat(mins, 16, axis=1)
    assert np.array_equal(got, (ds * q - dm).astype(np.float32))
    # unit scales: the codes themselves, in element order
    unit = both(Q.pack_q2_k(np.ones(blocks), np.zeros(blocks), np.ones((blocks, 16)), np.zeros((blocks, 16)), q),
                Q.Q2_K, blocks, 256, c_oracle)
    assert np.array_equal(unit, q.astype(np.float32))


def test_q3_k_scale_packing_exhaustive(c_oracle):
    """Every signed 6-bit scale in each of the 16 positions, codes -4..3 in every plane."""
    rng = np.random.default_rng(14)
    for index in range(16):
        blocks = 64
        scales = rng.integers(-32, 32, size=(blocks, 16))
        scales[:, index] = np.arange(-32, 32)
        q = np.ones((blocks, 256), dtype=np.int8)
        got = both(Q.pack_q3_k(np.ones(blocks), scales, q), Q.Q3_K, blocks, 256, c_oracle)
        assert np.array_equal(got, np.repeat(scales.astype(np.float32), 16, axis=1)), f"scale {index}"
    q = rng.integers(-4, 4, size=(64, 256)).astype(np.int8)
    q[0] = np.tile(np.arange(-4, 4), 32)
    unit = both(Q.pack_q3_k(np.ones(64), np.ones((64, 16)), q), Q.Q3_K, 64, 256, c_oracle)
    assert np.array_equal(unit, q.astype(np.float32))
    d = fp16(rng, 64)
    scales = rng.integers(-32, 32, size=(64, 16))
    got = both(Q.pack_q3_k(d, scales, q), Q.Q3_K, 64, 256, c_oracle)
    expected = d.astype(np.float64)[:, None] * np.repeat(scales, 16, axis=1) * q
    assert np.array_equal(got, expected.astype(np.float32))


def test_q5_k_fields(c_oracle):
    rng = np.random.default_rng(15)
    blocks = 256
    d, dmin = fp16(rng, blocks), fp16(rng, blocks)
    scales = rng.integers(0, 64, size=(blocks, 8))
    mins = rng.integers(0, 64, size=(blocks, 8))
    q = rng.integers(0, 32, size=(blocks, 256), dtype=np.uint8)
    got = both(Q.pack_q5_k(d, dmin, scales, mins, q), Q.Q5_K, blocks, 256, c_oracle)
    ds = d.astype(np.float64)[:, None] * np.repeat(scales, 32, axis=1)
    dm = dmin.astype(np.float64)[:, None] * np.repeat(mins, 32, axis=1)
    assert np.array_equal(got, (ds * q - dm).astype(np.float32))
    # the high bit alone: q = 16 * bit places bit 4 of element e in qh byte e % 32, bit e // 32
    bits = rng.integers(0, 2, size=(blocks, 256), dtype=np.uint8)
    unit = both(Q.pack_q5_k(np.ones(blocks), np.zeros(blocks), np.ones((blocks, 8)), np.zeros((blocks, 8)), 16 * bits),
                Q.Q5_K, blocks, 256, c_oracle)
    assert np.array_equal(unit, 16.0 * bits)


@pytest.mark.parametrize("t", MORE + TYPES)
def test_quantizers_reconstruct_their_input(t, c_oracle):
    """The seeded quantizers (encoder direction) and the decoders agree on what a block
    means: decoding a quantized matrix reproduces it within the format's resolution."""
    w = np.random.default_rng(16).standard_normal((16, 512)).astype(np.float32) * 0.02
    raw = Q.quantize(w, t)
    error = np.linalg.norm(both(raw, t, 16, 512, c_oracle) - w) / np.linalg.norm(w)
    bound = {Q.Q2_K: 0.4, Q.Q3_K: 0.2, Q.Q4_0: 0.12, Q.Q4_1: 0.12, Q.Q4_K: 0.12}.get(t, 0.06)
    assert error < bound, (Q.NAMES[t], error)


def test_all_zero_blocks_decode_to_zero(c_oracle):
    for t in TYPES + MORE:
        qk, size = Q.GEOMETRY[t]
        raw = np.zeros((4, size), dtype=np.uint8)
        assert not both(raw, t, 4, qk, c_oracle).any()


def test_row_major_block_order(c_oracle):
    """Block (n, b) sits at byte (n*K/QK + b)*BLOCK: permuting rows permutes output rows."""
    rng = np.random.default_rng(10)
    for t in TYPES + MORE:
        qk, size = Q.GEOMETRY[t]
        n, k = 6, 2 * 256
        raw = random_blocks(t, n * k // qk, rng).reshape(n, -1)
        base = both(raw, t, n, k, c_oracle)
        perm = rng.permutation(n)
        assert np.array_equal(both(raw[perm], t, n, k, c_oracle), base[perm])


def test_half_to_float_all_patterns(c_oracle):
    bits = np.arange(65536, dtype=np.uint32)
    f = np.array([c_oracle.lib.oracle_half_to_float(int(b)) for b in bits], dtype=np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rounding(c_oracle):
    rng = np.random.default_rng(11)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                        2.0 ** -14, 2.0 ** -14 - 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                        np.inf, -np.inf], dtype=np.float32)
    values = np.concatenate([
        special,
        rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),
    ])
    got = np.array([c_oracle.lib.oracle_float_to_half(float(v)) for v in values], dtype=np.uint16)
    ref = values.astype(np.float16).view(np.uint16)
    nan = np.isnan(values)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)


@pytest.mark.parametrize("t", TYPES)
def test_linear_against_textbook_product(t, c_oracle):
    rng = np.random.default_rng(12)
    n, k, m = 24, 512, 3
    raw = Q.sample_weight(n, k, t, seed=100 + t)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = R.dequantize(raw, t, n, k).astype(np.float64)
    exact = x.astype(np.float64) @ w.T
    got = c_oracle.linear(x, raw, t, n, k)
    assert R.relative_l2(got, exact) < 1e-6
    # brute force one output element with a Python loop
    acc = sum(float(x[1, i]) * float(w[5, i]) for i in range(k))
    assert abs(got[1, 5] - acc) <= 1e-5 * max(1.0, abs(acc))
    # prefill numerics: fp16-rounded operands
    pre = c_oracle.linear(x, raw, t, n, k, prefill=True)
    assert R.relative_l2(pre, R.gemm_reference(x, raw, t, n, k)) < 1e-6


def test_prefill_reference_differs_from_decode_reference():
    """The fp16 rounding of W is visible: the two oracles are not the same function."""
    raw = Q.sample_weight(64, 512, Q.Q4_K, seed=1)
    x = Q.sample_activation(2, 512, seed=2)
    a = R.gemv_reference(x, raw, Q.Q4_K, 64, 512)
    b = R.gemm_reference(x, raw, Q.Q4_K, 64, 512)
    assert 1e-6 < R.relative_l2(b, a) < 2e-3


def test_silu_closed_forms():
    """silu(g) = g * sigmoid(g): scipy's logistic, the odd-part identity silu(g) - silu(-g) = g,
    its limits and zero (no NaN where exp(-g) overflows)."""
    from scipy.special import expit

    g = np.linspace(-30.0, 30.0, 601)
    np.testing.assert_allclose(R.silu(g), g * expit(g), rtol=1e-13, atol=1e-300)
    np.testing.assert_allclose(R.silu(g) - R.silu(-g), g, rtol=0, atol=1e-12)
    assert R.silu(0.0) == 0.0
    assert R.silu(-1000.0) == 0.0 and R.silu(1000.0) == 1000.0


def test_swiglu_reference_composition(c_oracle):
    """silu of the gate product times the up product, against the C decoder and scipy: a swap of
    gate and up, or the gate taken from the wrong matrix, changes the result."""
    from scipy.special import expit

    n, k = 48, 512
    gate = Q.sample_weight(n, k, Q.Q4_K, seed=11)
    up = Q.sample_weight(n, k, Q.Q4_K, seed=12)
    x = Q.sample_activation(3, k, seed=13).astype(np.float32).astype(np.float64)
    g = x @ c_oracle.dequantize(gate, Q.Q4_K, n, k).astype(np.float64).T
    u = x @ c_oracle.dequantize(up, Q.Q4_K, n, k).astype(np.float64).T
    got = R.swiglu_reference(x, gate, up, Q.Q4_K, n, k)
    np.testing.assert_allclose(got, g * expit(g) * u, rtol=1e-12, atol=1e-15)
    swapped = R.swiglu_reference(x, up, gate, Q.Q4_K, n, k)
    assert R.relative_l2(swapped, got) > 0.1


def test_relative_l2_definition():
    e = np.array([3.0, 4.0])
    assert R.relative_l2(e + np.array([0.3, 0.4]), e) == pytest.approx(0.1)
    assert R.relative_l2(np.ones(2), np.zeros(2)) == pytest.approx(np.sqrt(2) / 1e-12)


def test_oracle_fp16_weights_round_twice(c_oracle):
    """The prefill oracle casts the fp32 dequantized weight to fp16 (the reference's order,
    triton_kernels.py:199-211): for a weight whose fp32 value is an fp16 tie although the
    exact value is not, that differs from rounding the exact value once."""
    d, dmin = np.array([11277], np.uint16).view(np.float16), np.array([4647], np.uint16).view(np.float16)
    raw = Q.pack_q4_k(d, dmin, np.full((1, 8), 9), np.full((1, 8), 23), np.full((1, 256), 15, np.uint8))
    fp32 = both(raw, Q.Q4_K, 1, 256, c_oracle)
    exact = float(d[0]) * 9 * 15 - float(dmin[0]) * 23
    assert float(fp32[0, 0]) != exact and np.float16(exact) == np.float16(8.5234375)
    assert np.all(fp32.astype(np.float16) == np.float16(8.53125))
    x = np.zeros((1, 256), np.float16)
    x[0, 5] = 1.0
    assert c_oracle.linear(x, raw, Q.Q4_K, 1, 256, prefill=True)[0, 0] == np.float32(8.53125)

