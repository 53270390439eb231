"""Pins the CPU restatement of the Q8_1-activation integer-dot GEMV (``oracle/q8_1_ref.py``).

GGML is not in the reference tree, so nothing here compares against GGML's own outputs; the
checks are what the format and the mathematics fix: the quantizer's defining properties, and
the integer-dot products against an fp64 product of independently decoded operands.  A planted
mistake in the dot products (a wrong Q4_0 offset, a dropped Q4_K min term, a misplaced Q6_K
scale) must fail that comparison.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from oracle import q8_1_ref as Q81
from tests import gguf_cases as cases

TYPES = {"q4_0": R.Q4_0, "q8_0": R.Q8_0, "q4_k": R.Q4_K, "q6_k": R.Q6_K}


def test_quantize_q8_1_block_properties():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 256)) * rng.uniform(0.01, 30, (3, 1))).astype(np.float32)
    x[1, 32:64] = 0.0                                   # an all-zero block
    q, d, s = Q81.quantize_q8_1(x)
    assert q.dtype == np.int8 and d.shape == (3, 8) and s.shape == (3, 8)
    blocks = x.reshape(3, 8, 32)
    qb = q.reshape(3, 8, 32).astype(np.int32)
    amax = np.abs(blocks).max(axis=2)
    d32 = amax / np.float32(127)
    assert np.array_equal(d, d32.astype(np.float16).astype(np.float32))
    nonzero = amax > 0
    # the largest element of every block takes the code +-127, the others stay inside
    peak = np.take_along_axis(qb, np.abs(blocks).argmax(axis=2)[:, :, None], axis=2)[:, :, 0]
    assert np.all(np.abs(peak[nonzero]) == 127) and np.abs(qb).max() <= 127
    # round trip within half a step of the fp32 scale
    err = np.abs(blocks - qb * d32[:, :, None])
    assert np.all(err <= d32[:, :, None] * 0.5 * (1 + 1e-6))
    # zero block: zero codes, zero scale and sum
    assert not qb[1, 1].any() and d[1, 1] == 0 and s[1, 1] == 0
    # s is the fp16 value of d * sum(q) with the fp32 d
    expect_s = (qb.sum(axis=2).astype(np.float32) * d32).astype(np.float16).astype(np.float32)
    assert np.array_equal(s, expect_s)


def test_quantize_q8_1_rounds_ties_away_from_zero():
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0                        # d = 1, 1 / d = 1: codes are x rounded
    x[0, 1:7] = [2.5, -2.5, 0.5, -0.5, 126.5, -1.5]
    q, d, _ = Q81.quantize_q8_1(x)
    assert d[0, 0] == 1.0
    assert q[0, :7].tolist() == [127, 3, -3, 1, -1, 127, -2]


@pytest.mark.parametrize("encoding", list(TYPES))
@pytest.mark.parametrize("m,n,k", [(1, 40, 512), (3, 17, 1024)])
def test_gemv_q8_1_matches_the_fp64_product_of_decoded_operands(encoding, m, n, k):
    code = TYPES[encoding]
    raw = cases.weight(n, k, encoding, 600 + m)
    x = cases.activation(m, k, 610 + m).astype(np.float32)
    got = Q81.gemv_q8_1(x, raw, code, n, k)
    exact = Q81.gemv_q8_1_exact(x, raw, code, n, k)
    scale = np.abs(exact).max()
    assert np.abs(got - exact).max() <= 2e-6 * scale * np.sqrt(k / 32), encoding
    # and it approximates the fp32 decode within the reference's GGML qualification
    assert R.relative_l2(got, R.gemv_reference(x, raw, code, n, k)) <= 0.02


def test_planted_mistakes_fail_the_fp64_check():
    """The comparison above is sensitive to each term of the dot products: the same formulas with
    one term changed (computed here, on the CPU) leave the fp64 product far behind."""
    k, n = 512, 24
    x = cases.activation(1, k, 620).astype(np.float32)
    q, dx, sx = Q81.quantize_q8_1(x)
    qb = q.reshape(1, k // 32, 32).astype(np.int64)

    def run(code, mutate):
        raw = cases.weight(n, k, {R.Q4_0: "q4_0", R.Q4_K: "q4_k", R.Q6_K: "q6_k"}[code], 630)
        codes, f = Q81._weight_blocks(raw, code, n, k)
        acc = np.zeros((1, n), np.float64)
        for b in range(k // 32):
            if code == R.Q6_K:
                prod = (codes[:, b, :] * qb[0, b]).reshape(n, 2, 16).sum(axis=2)
                sc = f["sc"][:, b, ::-1] if mutate else f["sc"][:, b]  # scales of the two groups swapped
                acc[0] += f["d"][:, b] * dx[0, b] * (prod * sc).sum(axis=1)
            else:
                isum = (codes[:, b, :] * qb[0, b]).sum(axis=1)
                if code == R.Q4_0:
                    offset = 7.0 if mutate else 8.0
                    acc[0] += f["d"][:, b] * (dx[0, b] * isum - offset * sx[0, b])
                else:
                    minus = 0.0 if mutate else (f["dmin"][:, b] * f["m"][:, b]) * sx[0, b]
                    acc[0] += (f["d"][:, b] * f["sc"][:, b]) * (dx[0, b] * isum) - minus
        return acc, Q81.gemv_q8_1_exact(x, raw, code, n, k)

    for code in (R.Q4_0, R.Q4_K, R.Q6_K):
        good, exact = run(code, False)
        bad, _ = run(code, True)
        assert R.relative_l2(good, exact) <= 1e-6, code
        assert R.relative_l2(bad, exact) >= 1e-3, code


def test_gemv_q8_1_zero_activations_give_zero():
    raw = cases.weight(8, 256, "q4_k", 640)
    out = Q81.gemv_q8_1(np.zeros((2, 256), np.float32), raw, R.Q4_K, 8, 256)
    assert np.array_equal(out, np.zeros_like(out))
