"""The seeded full-size inputs of the GPU parity tests can see row-mapping mistakes.

Tall weights are built from one quantized slab of ``gguf_cases.SLAB_ROWS`` rows.
These CPU tests plant, in the oracle's own output, the mistakes a kernel's row
or workgroup indexing could make, and check that the GPU tests' tolerance
rejects each of them.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q
from tests import gguf_cases as cases

TOLERANCE = 2e-3
SLAB = cases.SLAB_ROWS


@pytest.mark.parametrize("encoding", ["q4_k", "q6_k", "q8_0", "q4_0", "q5_k", "q3_k"])
def test_tall_weights_differ_from_their_repeats(encoding):
    n, k = 2 * SLAB + 300, 512
    raw = cases.weight(n, k, encoding, 5)
    same = np.all(raw[:n - SLAB] == raw[SLAB:], axis=1)
    assert same.mean() < 0.01, same.mean()
    # the quantized codes repeat; only the fp16 scale fields were changed
    qk, size = Q.GEOMETRY[Q.ggml_type(encoding)]
    slab = Q.sample_weight(SLAB, k, encoding, seed=5)
    keep = np.ones(size, bool)
    for offset in cases.HALF_FIELDS[Q.ggml_type(encoding)]:
        keep[offset:offset + 2] = False
    codes = raw.reshape(n, -1, size)[..., keep]
    assert np.array_equal(codes[:SLAB], slab.reshape(SLAB, -1, size)[..., keep])
    assert np.array_equal(codes[SLAB:2 * SLAB], codes[:SLAB])


@pytest.mark.parametrize("shift", [SLAB, 2 * SLAB, -SLAB])
def test_rows_read_one_slab_away_fail_the_tolerance(c_oracle, shift):
    """A kernel that reads weight row r + shift for output row r (a wrapped workgroup index)."""
    n, k = 3 * SLAB + 77, 1024
    code = Q.Q4_K
    raw = cases.weight(n, k, code, 9)
    x = cases.activation(1, k, 10)
    c_oracle.set_threads(8)
    expected = c_oracle.linear(x, raw, code, n, k)
    rows = (np.arange(n) + shift) % n
    wrong = c_oracle.linear(x, raw[rows], code, n, k)
    assert R.relative_l2(wrong, expected) > 50 * TOLERANCE

