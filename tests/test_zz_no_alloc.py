"""The grouped prefill GEMM on the library's static scratch (tensor_gguf_gemm_group_noalloc_v1)
against the same GEMM with a caller's workspace (tensor_gguf_gemm_group_v1), both called
through the C ABI: bit for bit, on two calls in a row, the second with a smaller input, so
that the second call runs on a scratch array that still holds the first call's partial sums.
Both calls split K across workgroups, so the scratch is where their partial sums go."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_ref as R
from tensor_amd.gguf import quant as Q
from tests import gguf_cases as cases

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # TENSOR_GGUF_NOALLOC_SCRATCH_BYTES
CALLS = (
    ("q4_k", 256, 4096, (4096, 1024, 1024)),  # C5 q + k + v: 4-way K split, 24 MiB of partial sums
    ("q6_k", 200, 8192, (300, 500, 64)),      # smaller and ragged, a different split
    ("q4_0", 32, 4096, (4096, 1024, 1024)),   # M <= 64: 64 x 64 tiles, 2-way K split, 1.5 MiB
)


def _run(device, kernel, encoding, x, raws, out_dtype, workspace_bytes):
    m = x.shape[0]
    rows = [raw.shape[0] for raw in raws]
    exe = device.load(kernel, encoding=encoding, out_dtype=out_dtype, count=len(raws))
    xb = device.from_numpy(x)
    wbs = [device.from_numpy(raw) for raw in raws]
    outs = [device.empty((m, n), out_dtype) for n in rows]
    args = [xb]
    for wb, out in zip(wbs, outs):
        device.fill_bytes(out, 0xFF)  # an element left unwritten reads as NaN
        args += [wb, out]
    extra = []
    if workspace_bytes is not None:
        workspace = device.empty((max(256, workspace_bytes),), "uint8")
        device.fill_bytes(workspace, 0xFF)
        extra = [workspace]
    exe.launch(*args, *extra)
    results = [out.to_numpy() for out in outs]
    for b in [xb, *wbs, *outs, *extra]:
        b.release()
    return results


@pytest.mark.parametrize("out_dtype", ["float32", "float16"])
def test_noalloc_matches_the_workspace_form_on_two_calls(hip_device, c_oracle, out_dtype):
    c_oracle.set_threads(16)
    for index, (encoding, m, k, rows) in enumerate(CALLS):
        print(f"[noalloc] call {index}: {encoding} m={m} k={k} rows={rows} {out_dtype}", flush=True)
        need = hip_device.gemm_workspace(encoding, m, k, list(rows))
        assert 0 < need <= SCRATCH_BYTES, need
        x = cases.activation(m, k, 900 + index)
        raws = [cases.weight(n, k, encoding, 910 + 10 * index + i) for i, n in enumerate(rows)]
        got = _run(hip_device, "gguf_gemm_group_noalloc", encoding, x, raws, out_dtype, None)
        want = _run(hip_device, "gguf_gemm_group", encoding, x, raws, out_dtype, need)
        for i, n in enumerate(rows):
            assert not np.isnan(got[i]).any(), (index, i)
            assert np.array_equal(got[i].view(np.uint8), want[i].view(np.uint8)), (index, i)
            if out_dtype == "float32":
                err = R.relative_l2(got[i], c_oracle.linear(x, raws[i], Q.ggml_type(encoding), n, k, prefill=True))
                assert err <= 1e-5, (index, i, err)


def test_noalloc_calls_on_two_streams_take_the_scratch_in_turn(c_oracle):
    """Eager calls on two sessions' streams, enqueued back to back with no host wait between
    them: the library orders each call after the previous one on the other stream, so both give
    the workspace form's bits although they share the scratch."""
    import tensor_amd as tx

    encoding, m, k, rows = CALLS[0]
    inputs = [(cases.activation(m, k, 950 + i), [cases.weight(n, k, encoding, 960 + 10 * i + j)
                                                 for j, n in enumerate(rows)]) for i in range(2)]
    with tx.Device(0, provider="hip") as first, tx.Device(0, provider="hip") as second:
        assert first.stream != second.stream
        sessions = (first, second)
        exes = [d.load("gguf_gemm_group_noalloc", encoding=encoding, out_dtype="float32", count=len(rows))
                for d in sessions]
        calls, keep = [], []
        for device, exe, (x, raws) in zip(sessions, exes, inputs):
            xb = device.from_numpy(x)
            wbs = [device.from_numpy(raw) for raw in raws]
            outs = [device.empty((m, n), "float32") for n in rows]
            args = [xb]
            for wb, out in zip(wbs, outs):
                device.fill_bytes(out, 0xFF)
                args += [wb, out]
            device.synchronize()
            calls.append(exe.bind(*args))
            keep.append((xb, wbs, outs))
        print("[noalloc] two streams, three alternating rounds", flush=True)
        for _ in range(3):
            calls[0].launch()
            calls[1].launch()
        for device in sessions:
            device.synchronize()
        got = [[out.to_numpy() for out in outs] for _, _, outs in keep]
        want = [_run(device, "gguf_gemm_group", encoding, x, raws, "float32",
                     device.gemm_workspace(encoding, m, k, list(rows)))
                for device, (x, raws) in zip(sessions, inputs)]
    for session in range(2):
        for i in range(len(rows)):
            assert not np.isnan(got[session][i]).any(), (session, i)
            assert np.array_equal(got[session][i].view(np.uint8), want[session][i].view(np.uint8)), (session, i)
