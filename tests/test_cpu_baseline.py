"""The CPU baseline's TensorKernelV1 entries (oracle/gguf_ref.c), called through the descriptor
bench.py builds, as the reference CPU provider calls a native image
(src/tensor/providers/cpu.py:153-197): the decode entry gives the oracle's decode numerics and the
prefill entry its prefill numerics, bit for bit, and both refuse a call for another device."""

from __future__ import annotations

import ctypes as c

import numpy as np
import pytest

import bench
from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q
from tensor_amd.runtime import abi
from tests import gguf_cases as cases


@pytest.fixture(scope="module")
def entries(c_oracle):
    for entry in (c_oracle.entry, c_oracle.gemm_entry):
        entry.argtypes = [c.POINTER(abi.CallDescriptor), c.POINTER(abi.ErrorDescriptor)]
        entry.restype = c.c_int32
    c_oracle.set_threads(4)
    return c_oracle


@pytest.mark.parametrize("encoding,m,out_dtype", [("q4_k", 3, np.float16), ("q6_k", 5, np.float32),
                                                  ("q8_0", 1, np.float16)])
def test_entries_match_the_oracle_numerics(entries, encoding, m, out_dtype):
    n, k = 40, 512
    code = Q.ggml_type(encoding)
    raw = cases.weight(n, k, encoding, 7)
    x = cases.activation(m, k, 8)
    for entry, prefill in ((entries.entry, False), (entries.gemm_entry, True)):
        out = np.full((m, n), np.nan, out_dtype)
        call, _keep = bench.cpu_call(x, raw, out, code)
        error = abi.ErrorDescriptor()
        assert entry(c.byref(call), c.byref(error)) == 0, error.message
        want = entries.linear(x, raw, code, n, k, prefill=prefill, out_dtype=out_dtype)
        assert np.array_equal(out.view(np.uint8), want.view(np.uint8)), (encoding, prefill)
    # the prefill entry rounds both operands to fp16 (benchmark.py:473-477)
    want = R.gemm_reference(x, raw, code, n, k)
    assert R.relative_l2(out.astype(np.float32), want) <= 2e-3


def test_entries_refuse_a_device_stream(entries):
    raw = cases.weight(16, 256, "q4_k", 9)
    x = cases.activation(1, 256, 10)
    out = np.empty((1, 16), np.float16)
    call, _keep = bench.cpu_call(x, raw, out, Q.Q4_K)
    call.stream = abi.StreamDescriptor(10, 0, 0)
    for entry in (entries.entry, entries.gemm_entry):
        error = abi.ErrorDescriptor()
        assert entry(c.byref(call), c.byref(error)) == 3
        assert b"synchronous CPU stream" in error.message
