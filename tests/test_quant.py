"""Host-side GGUF quantizers: format invariants and error bounds (CPU)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q


def test_q8_0_round_trip_bound():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((8, 1024)).astype(np.float32) * 0.02
    raw = Q.quantize(w, "q8_0")
    blocks = raw.reshape(-1, 34)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    deq = R.dequantize(raw, Q.Q8_0, 8, 1024).reshape(-1, 32)
    err = np.abs(deq - w.reshape(-1, 32))
    # rounding to the nearest code plus the fp16 rounding of d (relative 2^-11)
    bound = d[:, None] * (0.5 + 127 * 2.0 ** -11) + 1e-12
    assert np.all(err <= bound)


@pytest.mark.parametrize("name,limit", [("q4_0", 0.12), ("q8_0", 0.01), ("q4_k", 0.1), ("q6_k", 0.03)])
def test_gaussian_quantization_error(name, limit):
    code = Q.ggml_type(name)
    rng = np.random.Generator(np.random.PCG64(3))
    w = rng.standard_normal((32, 2048), dtype=np.float32) * np.float32(0.02)
    raw = Q.quantize(w, name)
    assert raw.shape == (32, Q.row_bytes(code, 2048))
    deq = R.dequantize(raw, code, 32, 2048)
    assert R.relative_l2(deq, w) < limit


def test_q4k_codes_and_scales_in_range():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((4, 512)).astype(np.float32)
    raw = Q.quantize(w, "q4_k").reshape(-1, 144)
    d = raw[:, 0:2].copy().view(np.float16)
    dmin = raw[:, 2:4].copy().view(np.float16)
    assert np.all(d >= 0) and np.all(dmin >= 0)


def test_sample_weight_is_chunk_invariant():
    a = Q.sample_weight(37, 512, "q6_k", seed=5, chunk_rows=7)
    b = Q.sample_weight(37, 512, "q6_k", seed=5)
    assert np.array_equal(a, b)


def test_sample_weight_deterministic_and_seeded():
    a = Q.sample_weight(8, 256, "q4_k", seed=1)
    assert np.array_equal(a, Q.sample_weight(8, 256, "q4_k", seed=1))
    assert not np.array_equal(a, Q.sample_weight(8, 256, "q4_k", seed=2))


def test_type_names_and_errors():
    assert Q.ggml_type("Q4_K") == 12 and Q.ggml_type(14) == 14 and Q.ggml_type("q5_k") == 13
    with pytest.raises(ValueError):
        Q.ggml_type("iq4_xs")
    with pytest.raises(ValueError):
        Q.ggml_type(15)
    with pytest.raises(ValueError):
        Q.row_bytes(Q.Q4_K, 300)
