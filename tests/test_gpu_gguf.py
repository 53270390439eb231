"""GPU parity of the HIP GGUF kernels against the CPU oracle, through the C ABI.

Every call goes Device.load -> Executable -> BoundCall -> TensorCallV1 ->
libtensor_hip.so.  Bars (BASELINE): dequantized weights bit-exact; GEMV and
GEMM outputs within relative L2 <= 2e-3 of the oracle (decode: fp32 operands,
benchmark.py:466-472; prefill: fp16-rounded operands, benchmark.py:473-477).
Input families follow the reference's qualification (benchmark.py:499-555):
random, the same input scaled by -1.5, zeros, outputs pre-filled with NaN, and
one captured graph replayed after its inputs change.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q
from tests import gguf_cases as cases

pytestmark = pytest.mark.gpu

TOLERANCE = 2e-3  # relative L2
# The showcase's encodings, then the other GGML formats (public layouts; generic kernels).
MORE = ("q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q5_k")
ENCODINGS = ("q4_k", "q6_k", "q8_0", "q4_0") + MORE


def note(*parts):
    print("[case]", *parts, flush=True)


def run_linear(device, kernel, encoding, x, raw, out_dtype):
    exe = device.load(kernel, encoding=encoding, out_dtype=out_dtype)
    xb, wb = device.from_numpy(x), device.from_numpy(raw)
    out = device.empty((x.shape[0], raw.shape[0]), out_dtype)
    device.fill_bytes(out, 0xFF)  # NaN in both fp16 and fp32
    exe.launch(xb, wb, out)
    result = out.to_numpy()
    for b in (xb, wb, out):
        b.release()
    return result


# ---------------------------------------------------------------- dequant --

@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("source", ["quantized", "random_bits"])
def test_dequant_bit_exact(hip_device, c_oracle, encoding, source):
    code = Q.ggml_type(encoding)
    n, k = 96, 3 * 256  # three super-blocks per row: odd Q6_K block alignment
    note("dequant", encoding, source, n, k)
    raw = cases.weight(n, k, encoding, 11) if source == "quantized" else cases.random_blocks(encoding, n, k, 12)
    expected = c_oracle.dequantize(raw, code, n, k)
    wb = hip_device.from_numpy(raw)
    for dtype in ("float32", "float16"):
        exe = hip_device.load("gguf_dequant", encoding=encoding, out_dtype=dtype)
        out = hip_device.empty((n, k), dtype)
        hip_device.fill_bytes(out, 0xFF)
        exe.launch(wb, out)
        got = out.to_numpy()
        want = expected if dtype == "float32" else expected.astype(np.float16)
        view = np.uint32 if dtype == "float32" else np.uint16
        assert np.array_equal(got.view(view), want.view(view)), f"{encoding} {dtype}"
        out.release()
    wb.release()


def test_dequant_fp16_subnormals(hip_device, c_oracle):
    """Tiny scales push decoded values into fp16's subnormal range; RNE must keep them."""
    n, k = 32, 512
    raw = cases.random_blocks("q4_k", n, k, 13, scale=2e-6)
    expected = c_oracle.dequantize(raw, Q.Q4_K, n, k).astype(np.float16)
    assert np.any((expected != 0) & (np.abs(expected) < np.float16(6.1e-5)))
    exe = hip_device.load("gguf_dequant", encoding="q4_k", out_dtype="float16")
    wb = hip_device.from_numpy(raw)
    out = exe(wb, K=k)
    assert np.array_equal(out.to_numpy().view(np.uint16), expected.view(np.uint16))
    out.release()
    wb.release()


# ------------------------------------------------------------------- GEMV --

@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("k", [2560, 8192])
def test_gemv_parity_small(hip_device, encoding, m, k):
    code = Q.ggml_type(encoding)
    n = 301  # ragged row count; K = 2560 is not a multiple of a full lane step
    note("gemv", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 20 + m)
    x = cases.activation(m, k, 30 + m)
    expected = R.gemv_reference(x, raw, code, n, k)
    for out_dtype in ("float32", "float16"):
        got = run_linear(hip_device, "gguf_gemv", encoding, x, raw, out_dtype)
        assert not np.isnan(got).any()
        err = R.relative_l2(got, expected)
        assert err <= TOLERANCE, (encoding, m, out_dtype, err)
        if out_dtype == "float32":
            assert err <= 2e-4, (encoding, m, err)


@pytest.mark.parametrize("encoding,n,k,m,out_dtype", [
    ("q4_k", 12288, 4096, 1, "float16"),   # C2 gate/up
    ("q4_k", 4096, 12288, 1, "float16"),   # C2 down
    ("q4_k", 12288, 4096, 4, "float16"),
    ("q4_k", 4096, 12288, 4, "float16"),   # C2 down at M = 4: one 16-row tile x 12 K ranges per workgroup
    ("q4_k", 12288, 4096, 8, "float16"),   # C2 gate at M = 8
    ("q4_k", 4096, 12288, 8, "float16"),   # C2 down at M = 8: K split into 4 ranges across workgroups
    ("q6_k", 151936, 4096, 1, "float32"),  # C3 LM head, fp32 logits
    ("q6_k", 4096, 12288, 1, "float16"),   # C5 down (Q6_K)
    ("q6_k", 1001, 12288, 1, "float32"),   # three steps per row, ragged last workgroup
    ("q8_0", 4096, 4096, 1, "float16"),    # C1 shape
    ("q8_0", 4096, 12288, 1, "float16"),   # six blocks per lane, 4-wave workgroups
    ("q4_0", 12288, 4096, 1, "float32"),
    ("q5_k", 12288, 4096, 1, "float16"),   # Q5_K through the M = 1 kernel (4 rows per workgroup)
    ("q5_k", 4096, 12288, 1, "float32"),   # three 4096-column steps, 8 rows per workgroup
    ("q5_k", 1003, 16384, 1, "float16"),   # four steps, ragged last workgroup
    ("q3_k", 12288, 4096, 1, "float16"),   # Q3_K / Q2_K through the per-sub-block M = 1 kernel
    ("q3_k", 4096, 12288, 1, "float32"),
    ("q2_k", 12288, 4096, 1, "float32"),
    ("q2_k", 4096, 12288, 1, "float16"),
    ("q4_k", 1536, 4096, 1, "float16"),    # one GPU's rows of an 8-way gate
    ("q4_k", 4096, 1536, 1, "float16"),    # one GPU's K slice of an 8-way down (generic kernel)
    ("q6_k", 4096, 1536, 1, "float16"),
    ("q6_k", 18992, 4096, 1, "float32"),   # one GPU's rows of an 8-way LM head
])
def test_gemv_parity_baseline_shapes(hip_device, c_oracle, encoding, n, k, m, out_dtype):
    code = Q.ggml_type(encoding)
    note("gemv-full", encoding, n, k, m, out_dtype)
    raw = cases.weight(n, k, encoding, 40)
    x = cases.activation(m, k, 41)
    c_oracle.set_threads(16)
    expected = c_oracle.linear(x, raw, code, n, k)
    got = run_linear(hip_device, "gguf_gemv", encoding, x, raw, out_dtype)
    assert R.relative_l2(got, expected) <= TOLERANCE


@pytest.mark.parametrize("encoding", ["q8_0", "q4_0"])
def test_gemv_q32_m1_every_row_length(hip_device, c_oracle, encoding):
    """M = 1 Q8_0 / Q4_0 rows of 2048 .. 16384 columns: one to eight blocks per lane, all held
    in registers, 8- and 4-wave workgroups, a ragged last workgroup (203 rows)."""
    code = Q.ggml_type(encoding)
    n = 203
    for k in range(2048, 16384 + 1, 2048):
        note("gemv-q32-m1", encoding, n, k)
        raw = cases.weight(n, k, encoding, 45 + k // 2048)
        x = cases.activation(1, k, 46)
        expected = c_oracle.linear(x, raw, code, n, k)
        for out_dtype in ("float32", "float16"):
            got = run_linear(hip_device, "gguf_gemv", encoding, x, raw, out_dtype)
            assert not np.isnan(got).any(), (k, out_dtype)
            err = R.relative_l2(got, expected)
            assert err <= (2e-4 if out_dtype == "float32" else TOLERANCE), (k, out_dtype, err)


@pytest.mark.parametrize("encoding", ["q4_1", "q5_0", "q5_1"])
@pytest.mark.parametrize("source", ["quantized", "random_bits"])
def test_gemv_q5_m1_every_row_length_each_row_within_tolerance(hip_device, c_oracle, encoding, source):
    """M = 1 Q4_1 / Q5_0 / Q5_1 rows of 2048 .. 16384 columns (one 32-element block per lane and
    one to eight blocks per lane, 8- and 4-wave workgroups, a ragged last workgroup of 203 rows;
    Q5_0's 22-byte blocks read through 4-byte-aligned windows), from quantized weights and from
    random block bytes (every fifth-bit pattern).  Each row is checked."""
    code = Q.ggml_type(encoding)
    n = 203
    for k in range(2048, 16384 + 1, 2048):
        note("gemv-q5-m1", encoding, source, n, k)
        raw = cases.weight(n, k, encoding, 51) if source == "quantized" else cases.random_blocks(encoding, n, k, 52)
        x = cases.activation(1, k, 53)
        expected = c_oracle.linear(x, raw, code, n, k)
        scale = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        for out_dtype in ("float32", "float16"):
            got = run_linear(hip_device, "gguf_gemv", encoding, x, raw, out_dtype)
            assert not np.isnan(got).any(), (k, out_dtype)
            assert R.relative_l2(got, expected) <= (2e-4 if out_dtype == "float32" else TOLERANCE), (k, out_dtype)
            err = np.abs(got[0].astype(np.float32) - expected[0])
            assert err.max() <= 2e-3 * scale + 1e-3 * np.abs(expected).max(), (k, out_dtype, int(err.argmax()))


@pytest.mark.parametrize("encoding", ["q2_k", "q3_k"])
@pytest.mark.parametrize("source", ["quantized", "random_bits"])
def test_gemv_q23k_m1_every_row_length_each_row_within_tolerance(hip_device, c_oracle, encoding, source):
    """M = 1 Q2_K / Q3_K rows of 4096 .. 16384 columns (the per-sub-block kernel: one to four
    4096-column steps, a ragged last workgroup of 203 rows), from quantized weights and from
    random block bytes (every scale, min and third-bit pattern in every position).  Each row is
    checked, so a misplaced plane, scale or run sum fails even where the whole output's
    relative L2 would hide it."""
    code = Q.ggml_type(encoding)
    n = 203
    for k in (4096, 8192, 12288, 16384):
        note("gemv-q23k-m1", encoding, source, n, k)
        raw = cases.weight(n, k, encoding, 47) if source == "quantized" else cases.random_blocks(encoding, n, k, 48)
        x = cases.activation(1, k, 49)
        expected = c_oracle.linear(x, raw, code, n, k)
        scale = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        for out_dtype in ("float32", "float16"):
            got = run_linear(hip_device, "gguf_gemv", encoding, x, raw, out_dtype)
            assert not np.isnan(got).any(), (k, out_dtype)
            assert R.relative_l2(got, expected) <= (2e-4 if out_dtype == "float32" else TOLERANCE), (k, out_dtype)
            err = np.abs(got[0].astype(np.float32) - expected[0])
            assert err.max() <= 2e-3 * scale + 1e-3 * np.abs(expected).max(), (k, out_dtype, int(err.argmax()))


@pytest.mark.parametrize("n", [65536 + 1007, 70000])
def test_gemv_q6k_tall_rows_each_within_tolerance(hip_device, c_oracle, n):
    """Tall K = 4096 Q6_K matrices (the LM head's shape class, ragged row counts): every row
    is checked, so a skipped, repeated or misplaced row fails even where the relative L2 of
    the whole output would hide it."""
    note("gemv-q6k-tall", n)
    k = 4096
    raw = cases.weight(n, k, "q6_k", 42)
    x = cases.activation(1, k, 43)
    c_oracle.set_threads(16)
    expected = c_oracle.linear(x, raw, Q.Q6_K, n, k)[0]
    scale = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
    for out_dtype in ("float32", "float16"):
        got = run_linear(hip_device, "gguf_gemv", "q6_k", x, raw, out_dtype)[0].astype(np.float32)
        assert not np.isnan(got).any()
        err = np.abs(got - expected)
        assert err.max() <= 2e-3 * scale + 1e-3 * np.abs(expected).max(), (out_dtype, int(err.argmax()))


@pytest.mark.parametrize("m,n,k", [
    (8, 8200, 4096),    # sector-aligned kernel, two tiles per workgroup, ragged last tile
    (6, 12296, 4096),   # sector-aligned, three tiles per workgroup, last workgroup one tile
    (3, 8200, 8192),    # sector-aligned, two tiles x eight K ranges (1024 threads)
    (4, 4101, 12288),   # sector-aligned for a long row, twelve K ranges, ragged rows
    (4, 4096, 12288),   # C2 down at M = 4: 256 workgroups, its 96 KB of x staged behind the weight loads
    (4, 12288, 4096),   # C2 gate at M = 4: 256 workgroups, 32 KB of x staged before the weight loads
    (2, 100, 16384),    # sector-aligned, sixteen K ranges of one 16-row tile
    (5, 4100, 12288),   # x too large for the sector kernel: K split into 4 ranges, 5 tiles per workgroup
    (8, 4100, 4096),    # narrow matrix: the LDS multi-tile kernel
    (3, 9000, 2560),    # K not a multiple of 1024: two tiles per wave, five waves
    (2, 40, 256),       # one super-block, one wave
    (4, 8200, 512),     # two tiles per wave and a single wave: the wave stores both tiles
    (8, 1024, 12288),   # x too large for LDS: K split into 4 ranges, 2 tiles per workgroup
    (8, 4100, 12288),   # C2 down at M = 8 with ragged rows: 4 ranges, 5 tiles per workgroup (208 workgroups)
    (4, 1000, 16384),   # the split at the smallest M it runs: 4 ranges, one tile per workgroup
    (6, 2000, 12288),   # 4 ranges, 2 tiles per workgroup, ragged last tile
    (7, 4096, 12288),   # 4 ranges at an odd row count: output rows past M in every tile
    (6, 300, 16384),    # the longest rows, x too large for LDS, too few tiles for a split: x per wave
    (8, 64, 16384),     # x of 256 KB
    (8, 300, 8448),     # K not a multiple of 1024 and x too large for LDS
])
def test_gemv_q4k_multirow_configurations(hip_device, m, n, k):
    code = Q.ggml_type("q4_k")
    note("gemv-multirow", m, n, k)
    raw = cases.weight(n, k, "q4_k", 80 + m)
    x = cases.activation(m, k, 90 + m)
    expected = R.gemv_reference(x, raw, code, n, k)
    for out_dtype in ("float16", "float32"):
        got = run_linear(hip_device, "gguf_gemv", "q4_k", x, raw, out_dtype)
        assert not np.isnan(got).any(), out_dtype
        err = R.relative_l2(got, expected)
        assert err <= TOLERANCE, (m, n, k, out_dtype, err)
        if out_dtype == "float32":
            assert err <= 2e-4, (m, n, k, err)


@pytest.mark.parametrize("encoding,m,k", [
    ("q4_k", 1, 4096),    # one launch of the grouped M = 1 kernel
    ("q4_k", 1, 12288),   # three 4096-column steps per row
    ("q4_k", 4, 4096),    # M > 1: two equal matrices in one multi-row launch, else one launch per matrix
    ("q6_k", 1, 4096),    # no grouped kernel: one launch per matrix
    ("q8_0", 2, 2560),
    ("q5_k", 1, 2048),
    ("q5_k", 1, 4096),    # the grouped M = 1 kernel with the fifth bits
])
@pytest.mark.parametrize("count", [1, 2, 3])
def test_gemv_group_parity(hip_device, encoding, m, k, count):
    """Grouped GEMV (x shared by up to three matrices) against the oracle, matrix by matrix."""
    code = Q.ggml_type(encoding)
    rows = (301, 77, 1040)[:count]  # ragged: the last workgroup of each matrix is partial
    note("gemv-group", encoding, m, k, rows)
    x = cases.activation(m, k, 60 + count)
    raws = [cases.weight(n, k, encoding, 61 + i) for i, n in enumerate(rows)]
    for out_dtype in ("float16", "float32"):
        exe = hip_device.load("gguf_gemv_group", encoding=encoding, out_dtype=out_dtype, count=count)
        xb = hip_device.from_numpy(x)
        wbs = [hip_device.from_numpy(r) for r in raws]
        outs = [hip_device.empty((m, n), out_dtype) for n in rows]
        args = [xb]
        for wb, out in zip(wbs, outs):
            hip_device.fill_bytes(out, 0xFF)
            args += [wb, out]
        exe.launch(*args)
        for i, (raw, out, n) in enumerate(zip(raws, outs, rows)):
            got = out.to_numpy()
            assert not np.isnan(got).any(), (i, out_dtype)
            err = R.relative_l2(got, R.gemv_reference(x, raw, code, n, k))
            assert err <= TOLERANCE, (encoding, i, out_dtype, err)
            if out_dtype == "float32":
                assert err <= 2e-4, (encoding, i, err)
        for b in [xb, *wbs, *outs]:
            b.release()


def test_gemv_group_matches_single_launches(hip_device):
    """gate + up as one grouped launch equals two gguf_gemv launches bit for bit."""
    k, rows = 4096, (12288, 12288)
    note("gemv-group-vs-single", rows, k)
    x = cases.activation(1, k, 70)
    raws = [cases.weight(n, k, "q4_k", 71 + i) for i, n in enumerate(rows)]
    group = hip_device.load("gguf_gemv_group", encoding="q4_k", out_dtype="float16", count=2)
    xb = hip_device.from_numpy(x)
    wbs = [hip_device.from_numpy(r) for r in raws]
    gate, up = group(xb, wbs[0], wbs[1])
    single = [run_linear(hip_device, "gguf_gemv", "q4_k", x, r, "float16") for r in raws]
    assert np.array_equal(gate.to_numpy().view(np.uint16), single[0].view(np.uint16))
    assert np.array_equal(up.to_numpy().view(np.uint16), single[1].view(np.uint16))
    for b in [xb, *wbs, gate, up]:
        b.release()


def run_swiglu(device, encoding, x, gate, up, out_dtype):
    exe = device.load("gguf_gemv_swiglu", encoding=encoding, out_dtype=out_dtype)
    xb, gb, ub = device.from_numpy(x), device.from_numpy(gate), device.from_numpy(up)
    out = device.empty((x.shape[0], gate.shape[0]), out_dtype)
    device.fill_bytes(out, 0xFF)  # NaN in both fp16 and fp32
    exe.launch(xb, gb, ub, out)
    result = out.to_numpy()
    for b in (xb, gb, ub, out):
        b.release()
    return result


@pytest.mark.parametrize("encoding,m,n,k", [
    ("q4_k", 1, 12288, 4096),   # C2 gate / up: the fused M = 1 kernel
    ("q4_k", 1, 1003, 8192),    # fused kernel, two column steps, ragged last workgroup
    ("q4_k", 1, 301, 2560),     # K not a multiple of 4096: generic gate / up pairs
    ("q4_k", 4, 301, 4096),     # M > 1: a gate tile and its up tile per workgroup (sector-aligned kernel)
    ("q4_k", 8, 12288, 4096),   # C2 gate / up at M = 8
    ("q4_k", 2, 1003, 8192),    # sixteen waves per workgroup, ragged last tile
    ("q4_k", 5, 77, 3072),      # three K ranges per tile
    ("q4_k", 3, 100, 2560),     # K not a multiple of 1024: generic pairs
    ("q6_k", 1, 300, 4096),
    ("q6_k", 3, 77, 512),
    ("q8_0", 2, 100, 2560),
    ("q4_0", 8, 65, 1024),
    ("q5_k", 1, 300, 2048),
    ("q5_k", 1, 1003, 8192),    # Q5_K through the fused M = 1 kernel
    ("q3_k", 3, 77, 512),
    ("q2_k", 1, 64, 4096),
    ("q4_1", 2, 100, 1024),
    ("q5_0", 4, 33, 512),
    ("q5_1", 8, 65, 1024),
])
def test_gemv_swiglu_parity(hip_device, encoding, m, n, k):
    """silu(x W_gate^T) * (x W_up^T) in one launch against the oracle's composition."""
    code = Q.ggml_type(encoding)
    note("gemv-swiglu", encoding, m, n, k)
    gate = cases.weight(n, k, encoding, 110 + m)
    up = cases.weight(n, k, encoding, 120 + m)
    x = cases.activation(m, k, 130 + m)
    expected = R.swiglu_reference(x, gate, up, code, n, k)
    for out_dtype in ("float16", "float32"):
        got = run_swiglu(hip_device, encoding, x, gate, up, out_dtype)
        assert not np.isnan(got).any(), out_dtype
        err = R.relative_l2(got, expected)
        assert err <= TOLERANCE, (encoding, m, out_dtype, err)
        if out_dtype == "float32":
            assert err <= 2e-4, (encoding, m, err)
    zero = run_swiglu(hip_device, encoding, np.zeros_like(x), gate, up, "float32")
    assert np.array_equal(zero, np.zeros_like(zero))


@pytest.mark.parametrize("encoding,m,k", [("q4_k", 1, 4096), ("q6_k", 1, 4096),
                                          ("q4_k", 8, 12288)])  # K split across workgroups + reduce
def test_gemv_input_families_and_graph_replay(hip_device, encoding, m, k):
    """One captured graph, replayed after x changes: random, x*-1.5, zeros."""
    code = Q.ggml_type(encoding)
    n = 1024
    note("gemv-graph", encoding, m, k)
    raw = cases.weight(n, k, encoding, 50)
    x = cases.activation(m, k, 51)
    exe = hip_device.load("gguf_gemv", encoding=encoding, out_dtype="float32")
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((m, n), "float32")
    call = exe.bind(xb, wb, out)
    graph = hip_device.graph(call.launch)
    try:
        for family, xs in (("random", x), ("fresh_scaled", (x.astype(np.float32) * -1.5).astype(np.float16)),
                           ("zero", np.zeros_like(x))):
            hip_device.upload(xb, xs)
            hip_device.fill_bytes(out, 0xFF)
            graph.replay()
            got = out.to_numpy()
            expected = R.gemv_reference(xs, raw, code, n, k)
            if family == "zero":
                assert np.array_equal(got, np.zeros_like(got)), family
            else:
                assert R.relative_l2(got, expected) <= TOLERANCE, family
    finally:
        graph.close()
        for b in (xb, wb, out):
            b.release()


def test_download_hooks_return_the_device_bytes(hip_device):
    """``_download_storage`` (the hook the reference's ``Buffer.to_bytes`` calls) and
    ``to_numpy`` / ``to_bytes`` give back the bytes uploaded, for a matrix and a view of it."""
    note("download-hooks")
    data = np.arange(3 * 40, dtype=np.float32).reshape(3, 40) * np.float32(-0.75)
    buffer = hip_device.from_numpy(data)
    stored = hip_device._download_storage(buffer)
    assert stored.dtype == np.float32 and stored.shape == (3, 40)
    assert np.array_equal(stored, data) and buffer.to_bytes() == data.tobytes()
    raw = hip_device.from_numpy(data.view(np.uint8).reshape(3, 160))
    assert np.array_equal(raw.view((480,)).to_numpy(), data.view(np.uint8).reshape(480))
    raw.release()
    buffer.release()


def test_graph_replay_refused_once_a_captured_buffer_is_released(hip_device):
    """A graph records the buffers of every call launched while it was captured (here through
    a lambda, so nothing is passed explicitly) and refuses to replay once one is released."""
    from tensor_amd._native import HipError

    note("graph-resources")
    raw, x = cases.weight(64, 256, "q4_k", 5), cases.activation(1, 256, 6)
    exe = hip_device.load("gguf_gemv", encoding="q4_k", out_dtype="float32")
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((1, 64), "float32")
    call = exe.bind(xb, wb, out)
    graph = hip_device.graph(lambda: call.launch())
    assert {id(b) for b in graph.resources} == {id(xb), id(wb), id(out)}
    graph.replay()
    expected = out.to_numpy()
    assert R.relative_l2(expected, R.gemv_reference(x, raw, Q.Q4_K, 64, 256)) <= TOLERANCE
    out.release()
    with pytest.raises(HipError, match="released resource"):
        graph.replay()
    out2 = hip_device.empty((1, 64), "float32")
    view = wb.view((64 * 144,))
    other = hip_device.graph(exe.bind(xb, wb, out2).launch, resources=(view,))
    other.replay()
    assert np.array_equal(out2.to_numpy(), expected)
    wb.release()  # releasing the base invalidates the base and the view the graph holds
    with pytest.raises(HipError, match="released resource"):
        other.replay()
    for g in (graph, other):
        g.close()
    for b in (xb, out2):
        b.release()


def test_linear_dispatch_matches_both_kernels(hip_device):
    n, k = 256, 1024
    raw = cases.weight(n, k, "q4_k", 60)
    for m in (1, 8, 9, 64):
        x = cases.activation(m, k, 61 + m)
        got = run_linear(hip_device, "gguf_linear", "q4_k", x, raw, "float32")
        expected = R.gemv_reference(x, raw, Q.Q4_K, n, k) if m <= 8 else R.gemm_reference(x, raw, Q.Q4_K, n, k)
        assert R.relative_l2(got, expected) <= TOLERANCE, m


# ------------------------------------------------------------------- GEMM --

@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("m", [1, 17, 128, 300])
def test_gemm_parity_small(hip_device, encoding, m):
    code = Q.ggml_type(encoding)
    n, k = 384 + 64, 1024
    note("gemm", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 70 + m)
    x = cases.activation(m, k, 80 + m)
    expected = R.gemm_reference(x, raw, code, n, k)
    for out_dtype in ("float32", "float16"):
        got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, out_dtype)
        assert not np.isnan(got).any()
        err = R.relative_l2(got, expected)
        assert err <= TOLERANCE, (encoding, m, out_dtype, err)
        if out_dtype == "float32":
            assert err <= 1e-5, (encoding, m, err)


@pytest.mark.parametrize("encoding,m,n,k", [
    ("q4_k", 512, 12288, 4096),   # C4
    ("q4_k", 2048, 12288, 4096),  # C4 at its larger M
    ("q6_k", 256, 4096, 12288),   # C5 down at M=256
    ("q8_0", 512, 12288, 4096),   # C4's shape in the showcase's other encodings
    ("q4_0", 512, 12288, 4096),
])
def test_gemm_parity_baseline_shapes(hip_device, c_oracle, encoding, m, n, k):
    """Full-size prefill shapes, every output row against the C oracle (16 threads)."""
    code = Q.ggml_type(encoding)
    note("gemm-full", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 90)
    x = cases.activation(m, k, 91)
    c_oracle.set_threads(16)
    expected = c_oracle.linear(x, raw, code, n, k, prefill=True)
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float16")
    assert not np.isnan(got).any()
    assert R.relative_l2(got, expected) <= TOLERANCE
    # row by row as well: a misplaced or skipped M tile hides in the L2 of the whole output
    rows = np.linalg.norm(got.astype(np.float32) - expected, axis=1) / np.linalg.norm(expected, axis=1)
    assert rows.max() <= 4 * TOLERANCE, int(rows.argmax())


@pytest.mark.parametrize("encoding,m,n,k", [
    ("q4_k", 512, 2304, 4096),    # 256 x 128 tiles, ragged last N tile
    ("q6_k", 300, 1000, 12288),   # K split inside the workgroup, ragged M and N
    ("q4_k", 1000, 12200, 512),   # 256 x 192 tiles, x by LDS DMA, ragged M and N
])
def test_gemm_input_families_and_graph_replay(hip_device, encoding, m, n, k):
    """The reference's prefill qualification (benchmark.py:499-555): one captured graph
    replayed after x changes (random, the same x * -1.5, zeros), out pre-filled with NaN
    before every replay."""
    code = Q.ggml_type(encoding)
    note("gemm-graph", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 150)
    x = cases.activation(m, k, 151)
    exe = hip_device.load("gguf_gemm", encoding=encoding, out_dtype="float16")
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((m, n), "float16")
    call = exe.bind(xb, wb, out)
    graph = hip_device.graph(call.launch)
    try:
        for family, xs in (("random", x), ("fresh_scaled", (x.astype(np.float32) * -1.5).astype(np.float16)),
                           ("zero", np.zeros_like(x))):
            hip_device.upload(xb, xs)
            hip_device.fill_bytes(out, 0xFF)
            graph.replay()
            got = out.to_numpy()
            assert not np.isnan(got).any(), family
            if family == "zero":
                assert np.array_equal(got, np.zeros_like(got)), family
            else:
                err = R.relative_l2(got, R.gemm_reference(xs, raw, code, n, k))
                assert err <= TOLERANCE, (family, err)
    finally:
        graph.close()
        for b in (xb, wb, out):
            b.release()


# Qwen3-8B decoder-layer linears (C5): name, encoding, N, K, which activation they read
C5_LAYER = (("q", "q4_k", 4096, 4096, "attn_in"), ("k", "q4_k", 1024, 4096, "attn_in"),
            ("v", "q4_k", 1024, 4096, "attn_in"), ("o", "q4_k", 4096, 4096, "attn_out"),
            ("gate", "q4_k", 12288, 4096, "mlp_in"), ("up", "q4_k", 12288, 4096, "mlp_in"),
            ("down", "q6_k", 4096, 12288, "mlp_mid"))


@pytest.mark.parametrize("m", [1, 256])
def test_c5_layer_chained_in_one_graph(hip_device, c_oracle, m):
    """C5: the seven linears of a Qwen3-8B decoder layer launched back to back on one
    stream from one captured graph, replayed twice, each output against the oracle.  At
    M = 1 the launches are the decode step's (q + k + v and gate + up grouped, since they
    share x); at M = 256 every linear is one prefill GEMM."""
    note("c5-layer", m)
    c_oracle.set_threads(16)
    widths = {"attn_in": 4096, "attn_out": 4096, "mlp_in": 4096, "mlp_mid": 12288}
    xs = {name: cases.activation(m, width, 300 + i) for i, (name, width) in enumerate(widths.items())}
    raws = {name: cases.weight(n, k, enc, 310 + i) for i, (name, enc, n, k, _) in enumerate(C5_LAYER)}
    xbs = {name: hip_device.from_numpy(x) for name, x in xs.items()}
    wbs = {name: hip_device.from_numpy(raw) for name, raw in raws.items()}
    outs = {name: hip_device.empty((m, n), "float16") for name, _, n, _, _ in C5_LAYER}
    calls = []
    if m == 1:
        qkv = hip_device.load("gguf_gemv_group", encoding="q4_k", out_dtype="float16", count=3)
        calls.append(qkv.bind(xbs["attn_in"], wbs["q"], outs["q"], wbs["k"], outs["k"], wbs["v"], outs["v"]))
        calls.append(hip_device.load("gguf_gemv", encoding="q4_k", out_dtype="float16")
                     .bind(xbs["attn_out"], wbs["o"], outs["o"]))
        pair = hip_device.load("gguf_gemv_group", encoding="q4_k", out_dtype="float16", count=2)
        calls.append(pair.bind(xbs["mlp_in"], wbs["gate"], outs["gate"], wbs["up"], outs["up"]))
        calls.append(hip_device.load("gguf_gemv", encoding="q6_k", out_dtype="float16")
                     .bind(xbs["mlp_mid"], wbs["down"], outs["down"]))
    else:
        # the prefill step: q + k + v and gate + up as grouped GEMMs (K split for q + k + v), o on
        # its own, the Q6_K down with its K split; one workspace, used by one launch at a time
        groups = [("attn_in", "q4_k", ("q", "k", "v")), ("attn_out", "q4_k", ("o",)),
                  ("mlp_in", "q4_k", ("gate", "up")), ("mlp_mid", "q6_k", ("down",))]
        rows = {name: n for name, _, n, _, _ in C5_LAYER}
        need = max(hip_device.gemm_workspace(enc, m, widths[src], [rows[n] for n in names])
                   for src, enc, names in groups)
        assert need > 0
        workspace = hip_device.empty((need,), "uint8")
        for src, enc, names in groups:
            exe = hip_device.load("gguf_gemm_group", encoding=enc, out_dtype="float16", count=len(names))
            args = [xbs[src]]
            for name in names:
                args += [wbs[name], outs[name]]
            calls.append(exe.bind(*args, workspace))
    graph = hip_device.graph(lambda: [call.launch() for call in calls])
    try:
        for replay in range(2):
            for out in outs.values():
                hip_device.fill_bytes(out, 0xFF)
            graph.replay()
            for name, enc, n, k, source in C5_LAYER:
                got = outs[name].to_numpy()
                assert not np.isnan(got).any(), (name, replay)
                expected = c_oracle.linear(xs[source], raws[name], Q.ggml_type(enc), n, k, prefill=m > 8)
                err = R.relative_l2(got, expected)
                assert err <= TOLERANCE, (name, replay, err)
    finally:
        graph.close()
        for b in {id(b): b for call in calls for b in call.buffers}.values():
            b.release()


@pytest.mark.parametrize("encoding", ["q4_k", "q5_k", "q6_k", "q8_0", "q4_0"])
@pytest.mark.parametrize("m,n,k", [
    (384, 7168, 512),    # 128x128 tile, K split over 2 wave groups
    (520, 4096, 512),    # 128x128, K split 2, ragged M
    (384, 7168, 768),    # 128x128 unsplit (12 K steps do not split evenly)
    (256, 9984, 768),    # 128x64 unsplit
    (80, 1000, 768),     # 64x64 unsplit, ragged N (M <= 64 at N <= 4096 takes the small-M kernel)
    (80, 1000, 512),     # 64x64, K split 2
    (256, 9984, 1024),   # 64x64, K split 4
    (300, 11000, 512),   # 256x96 (one round of 230 workgroups against 172 of 256x128), ragged M and N
    (512, 14000, 512),   # 256x128 (256x96 would need a second round)
    (1000, 12200, 512),  # 256x192 with x by LDS DMA for Q4_K / Q8_0 / Q4_0 (one round against two), ragged
])
def test_gemm_tile_configurations(hip_device, c_oracle, encoding, m, n, k):
    """Shapes that select each workgroup tile and K split of the prefill kernel."""
    code = Q.ggml_type(encoding)
    note("gemm-tiles", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 93)
    x = cases.activation(m, k, 94)
    c_oracle.set_threads(16)
    expected = c_oracle.linear(x, raw, code, n, k, prefill=True)
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float32")
    assert R.relative_l2(got, expected) <= 1e-5


@pytest.mark.parametrize("encoding,m,n,k", [
    ("q4_k", 96, 12288, 4096),    # 128 x 64 tiles, K over 2 wave groups (M <= 128)
    ("q6_k", 40, 20480, 1024),    # 64 x 64 tiles, K over 2 (M <= 64 and >= 256 tiles)
    ("q8_0", 100, 70000, 512),    # 128 x 128 unsplit (>= 512 tiles at M <= 128), ragged M and N
    ("q4_0", 130, 20480, 2048),   # 256 x 128 again from M = 129 (160 tiles)
])
def test_gemm_tiles_at_small_m(hip_device, c_oracle, encoding, m, n, k):
    """Tiles no more than twice as tall as M: shapes that select each of them below M = 129."""
    code = Q.ggml_type(encoding)
    note("gemm-small-m-tiles", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 95)
    x = cases.activation(m, k, 96)
    c_oracle.set_threads(16)
    expected = c_oracle.linear(x, raw, code, n, k, prefill=True)
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float32")
    rows = np.linalg.norm(got - expected, axis=1) / np.linalg.norm(expected, axis=1)
    assert rows.max() <= 1e-5, int(rows.argmax())


@pytest.mark.parametrize("encoding", ["q4_k", "q5_k", "q6_k", "q8_0", "q4_0"])
@pytest.mark.parametrize("k,n", [
    (512, 10240),   # 256x96 tile (214 workgroups in one round)
    (512, 14000),   # 256x128 tile, ragged N
    (1024, 2560),   # 128x128, K split 2
    (512, 1024),    # 64x64, K split 2
    (768, 320),     # 64x64 unsplit, ragged N
])
def test_gemm_one_hot_rows_give_dequantized_weights(hip_device, c_oracle, encoding, k, n):
    """Row m of x selects column perm[m] of W, so out[m, n] = fp16(dequant(W))[n, perm[m]]
    exactly: every staged weight of every code and scale is checked bit for bit."""
    code = Q.ggml_type(encoding)
    note("gemm-one-hot", encoding, k, n)
    raw = cases.random_blocks(encoding, n, k, 96)
    deq = c_oracle.dequantize(raw, code, n, k).astype(np.float16).astype(np.float32)
    perm = np.random.default_rng(97).permutation(k)
    x = np.zeros((k, k), np.float16)
    x[np.arange(k), perm] = 1.0
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float32")
    # the fp32 sum of one exact product and zeros is that product (a -0.0 weight reads +0.0)
    assert np.array_equal(got, deq[:, perm].T), encoding


@pytest.mark.parametrize("encoding", ["q4_k", "q8_0", "q4_0"])
@pytest.mark.parametrize("tile", [0, 8, 9])
def test_gemm_one_hot_rows_on_the_256_row_tiles(hip_device, c_oracle, encoding, tile):
    """The one-hot check through the plan entry on the 256-row tiles, the 256 x 192 LDS-DMA tile
    (half its waves multiply before they dequantize) among them: out[m, n] equals
    fp16(dequant(W))[n, perm[m]] bit for bit, at a ragged N."""
    k, n = 512, 1000
    code = Q.ggml_type(encoding)
    note("gemm-one-hot-256", encoding, tile)
    raw = cases.random_blocks(encoding, n, k, 98)
    deq = c_oracle.dequantize(raw, code, n, k).astype(np.float16).astype(np.float32)
    perm = np.random.default_rng(99).permutation(k)
    x = np.zeros((k, k), np.float16)
    x[np.arange(k), perm] = 1.0
    exe = hip_device.load("gguf_gemm_group_plan", encoding=encoding, out_dtype="float32", count=1)
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((k, n), "float32")
    workspace = hip_device.empty((256,), "uint8")
    hip_device.fill_bytes(out, 0xFF)
    exe.launch(xb, wb, out, workspace, tile=tile, splits=1)
    assert np.array_equal(out.to_numpy(), deq[:, perm].T), (encoding, tile)
    for buffer in (xb, wb, out, workspace):
        buffer.release()


@pytest.mark.parametrize("encoding,m,n,k,x_dtype", [
    ("q4_0", 2, 1000, 1056, "float32"),    # ragged N, a last half chunk of K (K % 64 == 32)
    ("q8_0", 33, 8200, 1056, "float32"),   # three M tiles, two 16-row tiles per workgroup
    ("q4_k", 64, 4096, 2048, "float16"),   # four M tiles, the widest N of the K-quants
    ("q6_k", 48, 1000, 4096, "float32"),
    ("q5_k", 16, 3000, 1024, "float16"),
    ("q2_k", 40, 9000, 768, "float32"),
    ("q3_k", 7, 2000, 768, "float16"),
    ("q4_1", 64, 8192, 1024, "float16"),
    ("q5_0", 20, 500, 1056, "float32"),
    ("q5_1", 3, 700, 1024, "float16"),
    ("q8_0", 3, 50, 32, "float32"),        # K = 32: one half chunk, only wave 0 has work
    ("q4_0", 9, 5, 96, "float16"),         # N < 16: every row index clamped, a half chunk
])
def test_gemm_small_m_kernel(hip_device, c_oracle, encoding, m, n, k, x_dtype):
    """M <= 64 (every encoding; the pipelined tiles keep N > 4096): weights decoded
    into MFMA operands, K over the waves of a workgroup, activations through a wave-private LDS
    tile.  Every output row against the prefill oracle (fp16 x and W, fp32 sums)."""
    note("gemm-small-m", encoding, m, n, k, x_dtype)
    check_packed_rows(hip_device, c_oracle, encoding, m, n, k, x_dtype, 600 + m)


@pytest.mark.parametrize("encoding,m,n,k,x_dtype", [
    ("q4_0", 32, 8192, 2048, "float16"),   # N > 4096: the pipelined tiles
    ("q8_0", 48, 6000, 1024, "float32"),   # pipelined, ragged M and N, fp32 x rounded as staged
    ("q8_0", 16, 6000, 1024, "float32"),   # Q8_0 with fp32 x at M <= 16: the small-M kernel
    ("q4_0", 20, 5000, 1056, "float16"),   # K % 64 == 32: the small-M kernel at any N
])
def test_gemm_small_m_at_wide_n(hip_device, c_oracle, encoding, m, n, k, x_dtype):
    """M <= 64 with N > 4096, on either side of the boundary between the small-M kernel and the
    pipelined tiles: every output row against the prefill oracle."""
    note("gemm-small-m-wide", encoding, m, n, k, x_dtype)
    check_packed_rows(hip_device, c_oracle, encoding, m, n, k, x_dtype, 650 + m)


def check_packed_rows(hip_device, c_oracle, encoding, m, n, k, x_dtype, seed):
    """The packed entry at (m, n, k), fp32 and fp16 out, every output row within tolerance."""
    code = Q.ggml_type(encoding)
    x, raw = showcase_inputs(encoding, m, n, k, seed)
    x = x.astype(x_dtype)
    expected = packed_reference(c_oracle, x, raw, code, m, n, k).reshape(m, n)
    for out_dtype in ("float32", "float16"):
        exe = hip_device.load("gguf_packed", encoding=encoding, m=m, n=n, k=k, x_dtype=x_dtype,
                              out_dtype=out_dtype)
        xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw.reshape(-1))
        out = hip_device.empty((m * n,), out_dtype)
        hip_device.fill_bytes(out, 0xFF)
        exe.launch(xb, wb, out)
        got = out.to_numpy().reshape(m, n).astype(np.float32)
        for b in (xb, wb, out):
            b.release()
        assert not np.isnan(got).any(), out_dtype
        rows = np.linalg.norm(got - expected, axis=1) / np.linalg.norm(expected, axis=1)
        # fp32 out: the operands are the oracle's, only the order of the fp32 sums differs
        assert rows.max() <= (1e-5 if out_dtype == "float32" else 4 * TOLERANCE), (out_dtype, int(rows.argmax()))


def test_gemm_zero_input_gives_exact_zero(hip_device):
    raw = cases.weight(128, 512, "q4_k", 95)
    x = np.zeros((64, 512), np.float16)
    got = run_linear(hip_device, "gguf_gemm", "q4_k", x, raw, "float32")
    assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_linear_on_weights_read_from_a_gguf_file(hip_device, c_oracle, encoding, tmp_path):
    """Raw rows ingested from a GGUF file (a read-only memory map) feed the kernels as is."""
    from tensor_amd.gguf import file as G

    code = Q.ggml_type(encoding)
    n, k = 300, 2048
    note("gguf-file", encoding, n, k)
    raw = cases.weight(n, k, encoding, 95)
    path = G.write(tmp_path / "model.gguf", {"blk.0.ffn_up.weight": (code, (k, n), raw)},
                   {"general.architecture": "qwen3"})
    x = cases.activation(3, k, 96)
    expected = c_oracle.linear(x, raw, code, n, k)
    with G.read(path) as gguf:
        rows = gguf.raw("blk.0.ffn_up.weight")
        got = run_linear(hip_device, "gguf_linear", encoding, x, rows, "float32")
        del rows
    assert R.relative_l2(got, expected) <= TOLERANCE


# A Q4_K / Q5_K element whose fp32 value is an fp16 rounding tie although the exact value
# is not: d = fp16 bits 11277, dmin = fp16 bits 4647, scale 9, min 23, code 15 gives the
# exact 8.5273432..., fp32 8.52734375 (the midpoint of fp16 8.5234375 and 8.53125), so the
# reference's order (fp32 dequantization, then a cast) stores 8.53125 and a single
# rounding of the exact value would store 8.5234375.
TIE_D, TIE_DMIN, TIE_SC, TIE_MN, TIE_Q, TIE_HALF = 11277, 4647, 9, 23, 15, 8.53125


def tie_blocks(encoding, n, k):
    blocks = n * k // 256
    d = np.full(blocks, TIE_D, np.uint16).view(np.float16)
    dmin = np.full(blocks, TIE_DMIN, np.uint16).view(np.float16)
    scales, mins = np.full((blocks, 8), TIE_SC), np.full((blocks, 8), TIE_MN)
    q = np.full((blocks, 256), TIE_Q, np.uint8)
    pack = Q.pack_q4_k if encoding == "q4_k" else Q.pack_q5_k
    return pack(d, dmin, scales, mins, q).reshape(n, -1)


@pytest.mark.parametrize("encoding", ["q4_k", "q5_k"])
def test_fp16_weights_are_the_cast_of_the_fp32_dequantization(hip_device, c_oracle, encoding):
    """Dequantizer fp16 output and the weights the pipelined GEMM stages in fp16 (Q4_K and
    Q5_K) round the fp32 value, not the exact value."""
    code = Q.ggml_type(encoding)
    n, k = 256, 512
    note("fp16-tie", encoding)
    raw = tie_blocks(encoding, n, k)
    assert np.all(c_oracle.dequantize(raw, code, n, k).astype(np.float16) == TIE_HALF)
    exe = hip_device.load("gguf_dequant", encoding=encoding, out_dtype="float16")
    wb = hip_device.from_numpy(raw)
    out = exe(wb, K=k)
    assert np.all(out.to_numpy() == TIE_HALF)
    out.release()
    wb.release()
    x = np.zeros((64, k), np.float16)
    x[np.arange(64), np.arange(64) * 7] = 1.0  # one-hot rows: out = fp16 weights
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float32")
    assert np.all(got == TIE_HALF), np.unique(got)


@pytest.mark.parametrize("encoding,k", [(e, 512) for e in MORE] + [
    ("q8_0", 544),    # 17 K steps: odd, so the pipelined kernel passes the shape on
    ("q4_0", 1056),   # K % 64 == 32
])
def test_generic_gemm_one_hot_rows_give_dequantized_weights(hip_device, c_oracle, encoding, k):
    """The generic GEMM stages every weight of the other encodings, and of Q8_0 / Q4_0 where K
    is not an even number of 64-element steps, as fp16(dequant): one-hot rows read them back
    bit for bit."""
    code = Q.ggml_type(encoding)
    n = 384
    note("gemm-one-hot-generic", encoding, k)
    raw = cases.random_blocks(encoding, n, k, 98)
    deq = c_oracle.dequantize(raw, code, n, k).astype(np.float16).astype(np.float32)
    perm = np.random.default_rng(99).permutation(k)
    x = np.zeros((k, k), np.float16)
    x[np.arange(k), perm] = 1.0
    got = run_linear(hip_device, "gguf_gemm", encoding, x, raw, "float32")
    assert np.array_equal(got, deq[:, perm].T), encoding


@pytest.mark.parametrize("m,n,k", [(4, 1003, 4096), (8, 12288, 4096), (2, 300, 8192), (3, 200, 2560)])
def test_gemv_group_pair_of_equal_matrices(hip_device, m, n, k):
    """Two Q4_K matrices of one shape at 2 <= M <= 4 (gate and up) in one grouped launch: the
    multi-row kernel with a tile of each per workgroup (M = 8 and K = 2560 take one launch per
    matrix)."""
    note("gemv-group-pair", m, n, k)
    x = cases.activation(m, k, 200 + m)
    raws = [cases.weight(n, k, "q4_k", 201 + i) for i in range(2)]
    for out_dtype in ("float16", "float32"):
        exe = hip_device.load("gguf_gemv_group", encoding="q4_k", out_dtype=out_dtype, count=2)
        xb = hip_device.from_numpy(x)
        wbs = [hip_device.from_numpy(r) for r in raws]
        outs = [hip_device.empty((m, n), out_dtype) for _ in range(2)]
        for out in outs:
            hip_device.fill_bytes(out, 0xFF)
        exe.launch(xb, wbs[0], outs[0], wbs[1], outs[1])
        for raw, out in zip(raws, outs):
            got = out.to_numpy()
            assert not np.isnan(got).any(), out_dtype
            err = R.relative_l2(got, R.gemv_reference(x, raw, Q.Q4_K, n, k))
            assert err <= TOLERANCE, (m, n, k, out_dtype, err)
        for b in [xb, *wbs, *outs]:
            b.release()


# ---------------------------------------------------------- packed form --

def showcase_inputs(encoding, m, n, k, seed):
    """The showcase's GGUF data (benchmark.py:453-464): x = randn(M*K) * 0.2 in fp32, the flat
    raw bytes of W, out fp32 [M*N]; here seeded numpy draws and this suite's quantizer."""
    x = (np.random.default_rng(seed).standard_normal(m * k, dtype=np.float32) * np.float32(0.2))
    raw = cases.weight(n, k, encoding, seed + 1)
    return x, raw


def packed_reference(c_oracle, x, raw, code, m, n, k):
    """GEMV: fp32 x times the fp32-decoded W (benchmark.py:466-472); M > 1: fp16-rounded x and W,
    fp32 accumulation (:473-477)."""
    return c_oracle.linear(x.reshape(m, k), raw, code, n, k, prefill=m > 1).reshape(-1)


@pytest.mark.parametrize("encoding", ["q4_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("m", [1, 32])
def test_showcase_packed_call_unchanged(hip_device, c_oracle, encoding, m):
    """The showcase's exact argument list [x fp32 (M*K,), w raw bytes (flat), out fp32 (M*N,)]
    (benchmark.py:460-464) on an executable specialised on (m, n, k), as AKAS's is
    (kernels.py:114-119), at the showcase's shapes N = K = 1024, M in {1, 32} (:122-126).
    Qualified as the showcase does (benchmark.py:499-555): one captured graph replayed after
    x changes (random, x * -1.5, zeros), out pre-filled with NaN before every replay."""
    n = k = 1024
    code = Q.ggml_type(encoding)
    note("packed", encoding, m, n, k)
    x, raw = showcase_inputs(encoding, m, n, k, 400 + m)
    exe = hip_device.load("gguf_linear", encoding=encoding, m=m, n=n, k=k)
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw.reshape(-1))
    out = hip_device.empty((m * n,), "float32")
    graph = hip_device.graph(exe.bind(xb, wb, out).launch)
    try:
        for family, xs in (("random", x), ("fresh_scaled", x * np.float32(-1.5)), ("zero", np.zeros_like(x))):
            hip_device.upload(xb, xs)
            hip_device.fill_bytes(out, 0xFF)
            graph.replay()
            got = out.to_numpy()
            assert not np.isnan(got).any(), family
            expected = packed_reference(c_oracle, xs, raw, code, m, n, k)
            if family == "zero":
                assert np.array_equal(got, np.zeros_like(got)), family
                continue
            err = R.relative_l2(got, expected)
            # fp32 operands at M = 1: only the accumulation order differs from the oracle
            assert err <= (1e-5 if m == 1 else TOLERANCE), (family, err)
    finally:
        graph.close()
        for b in (xb, wb, out):
            b.release()


@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("x_dtype,m", [("float32", 1), ("float16", 1), ("float32", 5), ("float16", 40)])
def test_packed_form_every_encoding(hip_device, c_oracle, encoding, x_dtype, m):
    """The packed entry for every encoding: fp32 x at M = 1 runs the fp32-operand GEMV, fp16 x
    at M = 1 the fp16 decode kernels, and M > 1 the prefill GEMM (x rounded to fp16 as it is
    staged), each against its oracle."""
    n, k = 300, 2048
    code = Q.ggml_type(encoding)
    note("packed-enc", encoding, x_dtype, m)
    x, raw = showcase_inputs(encoding, m, n, k, 500 + m)
    x = x.astype(x_dtype)
    for out_dtype in ("float32", "float16"):
        exe = hip_device.load("gguf_packed", encoding=encoding, m=m, n=n, k=k, x_dtype=x_dtype,
                              out_dtype=out_dtype)
        xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw.reshape(-1))
        out = hip_device.empty((m * n,), out_dtype)
        hip_device.fill_bytes(out, 0xFF)
        exe.launch(xb, wb, out)
        got = out.to_numpy()
        for b in (xb, wb, out):
            b.release()
        assert not np.isnan(got).any(), out_dtype
        expected = packed_reference(c_oracle, x, raw, code, m, n, k)
        err = R.relative_l2(got, expected)
        assert err <= TOLERANCE, (out_dtype, err)
        if m == 1 and x_dtype == "float32" and out_dtype == "float32":
            assert err <= 1e-5, err


@pytest.mark.parametrize("encoding,n,k", [
    ("q4_k", 1003, 4096),    # the fp32-x M = 1 kernel: one step, ragged last workgroup
    ("q4_k", 777, 12288),    # three steps (C2's down row length)
    ("q5_k", 500, 8192),
    ("q5_k", 100, 16384),    # four steps
    ("q6_k", 1001, 4096),    # LM-head row length
    ("q6_k", 300, 12288),
    ("q8_0", 1003, 4096),    # C1's row length
    ("q8_0", 257, 12288),
    ("q4_0", 300, 6144),
    ("q4_0", 1024, 1024),    # the showcase's row length: 32 blocks, half of each wave's lanes
    ("q8_0", 1001, 1024),
])
def test_packed_form_fp32_x_at_decode_row_lengths(hip_device, c_oracle, encoding, n, k):
    """fp32 x at M = 1 on the packed entry at the BASELINE row lengths, where the tuned decode
    kernels take the fp32 activations themselves: every row within tolerance of the fp32-operand
    oracle (benchmark.py:466-472), fp32 and fp16 out."""
    code = Q.ggml_type(encoding)
    note("packed-f32x", encoding, n, k)
    x, raw = showcase_inputs(encoding, 1, n, k, 700 + k // 1024)
    expected = packed_reference(c_oracle, x, raw, code, 1, n, k)
    for out_dtype in ("float32", "float16"):
        exe = hip_device.load("gguf_packed", encoding=encoding, m=1, n=n, k=k, out_dtype=out_dtype)
        xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw.reshape(-1))
        out = hip_device.empty((n,), out_dtype)
        hip_device.fill_bytes(out, 0xFF)
        exe.launch(xb, wb, out)
        got = out.to_numpy().astype(np.float32)
        for b in (xb, wb, out):
            b.release()
        assert not np.isnan(got).any(), out_dtype
        # fp32 operands: only the summation order differs from the oracle's k-order sums
        assert R.relative_l2(got, expected) <= (1e-5 if out_dtype == "float32" else TOLERANCE), out_dtype
        err = np.abs(got - expected)
        scale = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        bound = (1e-4 if out_dtype == "float32" else 2e-3) * scale + (0 if out_dtype == "float32" else 1e-3) * np.abs(expected)
        assert (err <= bound).all(), (out_dtype, int(np.argmax(err - bound)))


# ------------------------------------------------------- grouped prefill --

def run_gemm_group(device, encoding, x, raws, out_dtype, workspace_bytes=None):
    """gguf_gemm_group over matrices sharing x; workspace as the library asks, or the given size."""
    m, k = x.shape
    rows = [raw.shape[0] for raw in raws]
    need = device.gemm_workspace(encoding, m, k, rows)
    size = max(256, need if workspace_bytes is None else workspace_bytes)
    exe = device.load("gguf_gemm_group", encoding=encoding, out_dtype=out_dtype, count=len(raws))
    xb = device.from_numpy(x)
    wbs = [device.from_numpy(raw) for raw in raws]
    outs = [device.empty((m, n), out_dtype) for n in rows]
    workspace = device.empty((size,), "uint8")
    device.fill_bytes(workspace, 0xFF)  # stale partial sums would show up as NaN
    args = [xb]
    for wb, out in zip(wbs, outs):
        device.fill_bytes(out, 0xFF)
        args += [wb, out]
    exe.launch(*args, workspace)
    results = [out.to_numpy() for out in outs]
    for b in [xb, *wbs, *outs, workspace]:
        b.release()
    return results, need


@pytest.mark.parametrize("encoding,m,k,rows,split", [
    ("q4_k", 256, 4096, (4096, 1024, 1024), True),   # C5 q + k + v: K split over 4 workgroups
    ("q4_k", 256, 4096, (12288, 12288), False),      # C5 gate + up: one launch, 256 x 128 tiles
    ("q6_k", 256, 12288, (4096,), True),             # C5 down: K split over 8 workgroups
    ("q4_k", 256, 4096, (4096,), False),             # o: 64 x 64 tiles with the K range inside the workgroup
    ("q5_k", 300, 8192, (1000, 77), True),           # ragged M and N, Q5_K
    ("q6_k", 200, 8192, (300, 500, 64), True),       # three ragged matrices, K >= 8192
    ("q8_0", 64, 1024, (300, 100), False),           # small M: one small-M launch per matrix
    ("q8_0", 256, 12288, (4096,), True),             # Q8_0 down at M=256: K split across workgroups
    ("q4_0", 256, 4096, (4096, 1024, 1024), True),   # Q4_0 q + k + v in one split launch
    ("q4_0", 200, 1056, (300, 500), False),          # K % 64 == 32: one generic launch per matrix
    ("q4_k", 32, 4096, (4096, 1024, 1024), True),    # q + k + v at M=32: 64 x 64 tiles, K split 2 ways
    ("q6_k", 48, 12288, (4096,), True),              # down at M=48: 64 x 64 tiles, K split 4 ways
    ("q4_0", 16, 4096, (4096, 1024, 1024), True),    # Q4_0 q + k + v at M=16
    ("q6_k", 48, 2048, (3000, 100), False),          # small M, 98 workgroups at most: small-M kernel per matrix
    ("q4_k", 32, 1024, (1024,), False),              # the showcase's shape: small-M kernel
    ("q8_0", 100, 12288, (4096,), True),             # down at M=100: 256 x 128 tiles, K split 8 ways
    ("q4_k", 32, 4096, (12288, 12288), False),       # gate + up at M=32: 64 x 64 tiles, K over 2 wave groups
    ("q4_k", 128, 4096, (12288, 12288), False),      # gate + up at M=128: 128 x 128 tiles, K over 2
    ("q4_k", 160, 4096, (4096, 1024, 1024), True),   # q + k + v at M=160: K split 4 ways
])
def test_gemm_group_parity(hip_device, c_oracle, encoding, m, k, rows, split):
    code = Q.ggml_type(encoding)
    note("gemm-group", encoding, m, k, rows)
    x = cases.activation(m, k, 700 + len(rows))
    raws = [cases.weight(n, k, encoding, 710 + i) for i, n in enumerate(rows)]
    c_oracle.set_threads(16)
    for out_dtype in ("float16", "float32"):
        got, need = run_gemm_group(hip_device, encoding, x, raws, out_dtype)
        assert (need > 0) == split, need
        for i, (raw, n) in enumerate(zip(raws, rows)):
            assert not np.isnan(got[i]).any(), (i, out_dtype)
            err = R.relative_l2(got[i], c_oracle.linear(x, raw, code, n, k, prefill=True))
            assert err <= (TOLERANCE if out_dtype == "float16" else 1e-5), (i, out_dtype, err)


def test_gemm_group_with_a_short_workspace_splits_less(hip_device, c_oracle):
    """A workspace shorter than the plan wants limits the split (here to none, or to 2) and the
    result stays within tolerance of the same oracle."""
    m, k, rows = 256, 12288, (4096,)
    x = cases.activation(m, k, 720)
    raws = [cases.weight(rows[0], k, "q6_k", 721)]
    expected = c_oracle.linear(x, raws[0], Q.Q6_K, rows[0], k, prefill=True)
    for size in (256, 2 * m * rows[0] * 4):
        note("gemm-group-short-workspace", size)
        got, need = run_gemm_group(hip_device, "q6_k", x, raws, "float32", workspace_bytes=size)
        assert need > size
        assert R.relative_l2(got[0], expected) <= 1e-5


@pytest.mark.parametrize("encoding", ["q4_0", "q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("m,n,k,x_dtype", [
    (1, 1003, 4096, "float32"),   # ragged workgroup of rows
    (3, 777, 2560, "float16"),    # fp16 activations, K not a multiple of 1024
    (8, 300, 12288, "float32"),   # the most x the workgroup quantizes in LDS (M * K = 98304)
    (1, 12288, 4096, "float32"),  # C2 gate / up
    (1, 4096, 12288, "float16"),  # C2 / C5 down
    (4, 20001, 512, "float16"),   # several rows per wave, the last waves one row short
])
def test_gemv_q8_1_parity(hip_device, c_oracle, encoding, m, n, k, x_dtype):
    """The Q8_1-activation integer-dot GEMV against its CPU restatement (the same quantized
    codes, integer sums exact, fp32 scaling up to summation order: rel-L2 <= 1e-5 and every
    element within 2e-5 of the largest) and against the fp32 decode within the reference's GGML
    qualification (rel-L2 <= 0.02, external_baselines.py:53)."""
    from oracle import q8_1_ref as Q81

    code = Q.ggml_type(encoding)
    note("gemv-q8_1", encoding, m, n, k, x_dtype)
    raw = cases.weight(n, k, encoding, 700 + m)
    x = cases.activation(m, k, 710 + m).astype(x_dtype)
    expected = Q81.gemv_q8_1(x.astype(np.float32), raw, code, n, k)
    exe = hip_device.load("gguf_gemv_q8_1", encoding=encoding, out_dtype="float32", x_dtype=x_dtype)
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((m, n), "float32")
    hip_device.fill_bytes(out, 0xFF)
    exe.launch(xb, wb, out)
    got = out.to_numpy()
    assert not np.isnan(got).any()
    assert R.relative_l2(got, expected) <= 1e-5
    assert np.abs(got - expected).max() <= 2e-5 * np.abs(expected).max()
    c_oracle.set_threads(16)
    assert R.relative_l2(got, c_oracle.linear(x.astype(np.float32), raw, code, n, k)) <= 0.02
    out16 = hip_device.empty((m, n), "float16")
    hip_device.load("gguf_gemv_q8_1", encoding=encoding, out_dtype="float16", x_dtype=x_dtype).launch(xb, wb, out16)
    assert np.array_equal(out16.to_numpy(), got.astype(np.float16))
    for buffer in (xb, wb, out, out16):
        buffer.release()


@pytest.mark.parametrize("encoding,m,n,k", [("q8_0", 1, 1, 32), ("q4_0", 2, 3, 64), ("q4_k", 2, 65, 256),
                                            ("q6_k", 3, 9, 512)])
def test_gemv_q8_1_edge_shapes_and_zero_blocks(hip_device, encoding, m, n, k):
    """The smallest rows (one Q8_1 block, lane 0 alone), single output rows and activation rows
    with all-zero blocks (d = 0, codes 0): equal to the CPU restatement, zero rows exactly zero."""
    from oracle import q8_1_ref as Q81

    code = Q.ggml_type(encoding)
    note("gemv-q8_1-edges", encoding, m, n, k)
    raw = cases.weight(n, k, encoding, 720)
    x = cases.activation(m, k, 721).astype(np.float32)
    x[0, :32] = 0.0                    # a zero block in the first row
    if m > 1:
        x[1] = 0.0                     # and a zero row
    expected = Q81.gemv_q8_1(x, raw, code, n, k)
    exe = hip_device.load("gguf_gemv_q8_1", encoding=encoding, out_dtype="float32", x_dtype="float32")
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((m, n), "float32")
    hip_device.fill_bytes(out, 0xFF)
    exe.launch(xb, wb, out)
    got = out.to_numpy()
    assert not np.isnan(got).any()
    assert np.abs(got - expected).max() <= 2e-5 * max(np.abs(expected).max(), 1e-30)
    if m > 1:
        assert np.array_equal(got[1], np.zeros(n, np.float32))
    for buffer in (xb, wb, out):
        buffer.release()


def test_gemv_k_split_calls_on_two_streams_take_the_scratch_in_turn():
    """The multi-row GEMV plan that splits K across workgroups keeps its partial sums in the
    library's scratch: eager calls on two sessions' streams, enqueued back to back with no host
    wait between them, are ordered one after the other by the library, so each gives the bits
    it gives alone."""
    import tensor_amd as tx

    m, n, k = 8, 1000, 12288
    note("gemv-split-two-streams", m, n, k)
    inputs = [(cases.activation(m, k, 1600 + i), cases.weight(n, k, "q4_k", 1610 + i)) for i in range(2)]
    with tx.Device(0, provider="hip") as first, tx.Device(0, provider="hip") as second:
        assert first.stream != second.stream
        assert first.gemv_plan("q4_k", m, k, n)["name"] == "sec_split"
        sessions = (first, second)
        alone = [run_linear(device, "gguf_gemv", "q4_k", x, raw, "float32")
                 for device, (x, raw) in zip(sessions, inputs)]
        calls, outs, keep = [], [], []
        for device, (x, raw) in zip(sessions, inputs):
            exe = device.load("gguf_gemv", encoding="q4_k", out_dtype="float32")
            xb, wb, out = device.from_numpy(x), device.from_numpy(raw), device.empty((m, n), "float32")
            device.fill_bytes(out, 0xFF)
            calls.append(exe.bind(xb, wb, out))
            outs.append(out)
            keep += [xb, wb]
            device.synchronize()
        for _ in range(3):
            calls[0].launch()
            calls[1].launch()
        for device in sessions:
            device.synchronize()
        for session in range(2):
            got = outs[session].to_numpy()
            assert np.array_equal(got.view(np.uint32), alone[session].view(np.uint32)), session


@pytest.mark.parametrize("m,n,k", [(4, 2000, 4096), (3, 777, 8192), (8, 1000, 12288), (2, 40, 1280)])
def test_gemv_every_multirow_plan_through_the_variant_entry(hip_device, c_oracle, m, n, k):
    """Every multi-row Q4_K plan the variant entry accepts at ragged shapes (fp32 out): each within
    2e-4 of the decode oracle and within 1e-5 of the library plan's result; plans that do not fit
    are refused with an argument error before any launch, and the library's own plan is one of
    those that run."""
    from tensor_amd._native import HipError
    from tensor_amd.providers.hip import GEMV_FIELDS

    code = Q.ggml_type("q4_k")
    note("gemv-plans", m, n, k)
    raw, x = cases.weight(n, k, "q4_k", 1400 + m), cases.activation(m, k, 1410 + m)
    expected = c_oracle.linear(x, raw, code, n, k)
    library = hip_device.gemv_plan("q4_k", m, k, n)
    baseline = run_linear(hip_device, "gguf_gemv", "q4_k", x, raw, "float32")
    assert R.relative_l2(baseline, expected) <= 2e-4
    exe = hip_device.load("gguf_gemv_variant", encoding="q4_k", out_dtype="float32")
    xb, wb = hip_device.from_numpy(x), hip_device.from_numpy(raw)
    out = hip_device.empty((m, n), "float32")
    ran = []
    for kernel, fields in GEMV_FIELDS.items():
        for a, b in fields:
            hip_device.fill_bytes(out, 0xFF)
            try:
                exe.launch(xb, wb, out, kernel=kernel, a=a, b=b)
            except HipError as exc:
                assert exc.code == 2, (kernel, a, b, exc)
                continue
            ran.append((kernel, a, b))
            got = out.to_numpy()
            assert not np.isnan(got).any(), (kernel, a, b)
            assert R.relative_l2(got, expected) <= 2e-4, (kernel, a, b)
            assert R.relative_l2(got, baseline) <= 1e-5, (kernel, a, b)
    assert (library["kernel"], library["a"], library["b"]) in ran, (library, ran)
    assert len(ran) >= 2, ran
    for buffer in (xb, wb, out):
        buffer.release()


@pytest.mark.parametrize("encoding", ["q4_k", "q6_k", "q8_0", "q4_0"])
def test_gemm_every_plan_through_the_plan_entry(hip_device, c_oracle, encoding):
    """Every tile and K split the plan-naming entry accepts at a ragged grouped shape (two
    matrices, fp32 out): each within 1e-5 of the prefill oracle; plans that do not fit are
    refused with an argument error before any launch."""
    from tensor_amd._native import HipError
    from tensor_amd.providers.hip import gemm_tiles

    m, k, rows = 300, 1024, (2000, 1000)
    code = Q.ggml_type(encoding)
    note("gemm-plans", encoding, m, k, rows)
    raws = [cases.weight(n, k, encoding, 1300 + i) for i, n in enumerate(rows)]
    x = cases.activation(m, k, 1310)
    c_oracle.set_threads(16)
    expected = [c_oracle.linear(x, raw, code, n, k, prefill=True) for raw, n in zip(raws, rows)]
    exe = hip_device.load("gguf_gemm_group_plan", encoding=encoding, out_dtype="float32", count=2)
    xb = hip_device.from_numpy(x)
    wbs = [hip_device.from_numpy(raw) for raw in raws]
    outs = [hip_device.empty((m, n), "float32") for n in rows]
    workspace = hip_device.empty((4 * m * sum(rows) * 4,), "uint8")
    ran = 0
    for tile in range(len(gemm_tiles())):
        for splits in (1, 2, 4):
            for out in outs:
                hip_device.fill_bytes(out, 0xFF)
            try:
                exe.launch(xb, wbs[0], outs[0], wbs[1], outs[1], workspace, tile=tile, splits=splits)
            except HipError as exc:
                assert exc.code == 2, (tile, splits, exc)
                continue
            ran += 1
            for i, out in enumerate(outs):
                got = out.to_numpy()
                assert not np.isnan(got).any(), (tile, splits, i)
                assert R.relative_l2(got, expected[i]) <= 1e-5, (tile, splits, i)
    assert ran >= 12, ran
    for b in [xb, *wbs, *outs, workspace]:
        b.release()
