"""PyTorch-ROCm interop checks, run as its own process by test_gpu_torch.py.

torch is imported before anything loads libtensor_hip.so, so the library binds
to the HIP runtime that torch's wheel carries and the two share streams and
pointers.  Each check prints its name before it touches the GPU.
"""

from __future__ import annotations

import gc
import os
import sys
import time
from pathlib import Path

import torch  # first: the process's HIP runtime is torch's

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

import tensor_amd.torch as tt  # noqa: E402
from oracle import gguf_ref as R  # noqa: E402
from tensor_amd.gguf import quant as Q  # noqa: E402
from tensor_amd.runtime.errors import TensorRuntimeError  # noqa: E402
from tensor_amd.torch import launch as L  # noqa: E402
from tensor_amd.torch import session as S  # noqa: E402
from tests import gguf_cases as cases  # noqa: E402

TOLERANCE = 2e-3  # relative L2 against the oracle


def step(name):
    print("[torch-interop]", name, flush=True)


def check_linear(oracle, encoding, m, n, k, out_dtype, seed=60):
    step(f"linear {encoding} M={m} N={n} K={k} {out_dtype}")
    code = Q.ggml_type(encoding)
    raw, x = cases.weight(n, k, encoding, seed), cases.activation(m, k, seed + 1)
    kernel = tt.load("gguf_linear", encoding=encoding, out_dtype=out_dtype)
    xt, wt = torch.from_numpy(x).cuda(), torch.from_numpy(raw).cuda()
    out = kernel(xt, wt)
    assert out.shape == (m, n) and out.dtype == getattr(torch, out_dtype) and out.device == xt.device
    expect(oracle, out, x, raw, code, n, k)
    # same shapes, new storage: the cached descriptors are rebound to the new pointers
    x2 = (x * np.float16(-1.5)).astype(np.float16)
    out2 = kernel(torch.from_numpy(x2).cuda(), wt.clone())
    expect(oracle, out2, x2, raw, code, n, k)
    assert len(kernel._prepared) == 1
    assert len(kernel._plans) == (1 if L.native_executor() else 0)  # the second call ran the plan
    return kernel, xt, wt, out


def check_misaligned_weights():
    """Weights at a 2-byte storage offset are refused before any launch.  The M = 1 kernels of
    Q8_0, Q4_0, Q6_K, Q3_K and Q5_0 read their 2-mod-4 blocks through 4-byte-aligned windows,
    which the entry points' 16-byte buffer alignment guarantees."""
    for encoding in ("q8_0", "q6_k", "q3_k"):
        step(f"misaligned weights {encoding}: refused")
        raw, x = cases.weight(64, 4096, encoding, 80), cases.activation(1, 4096, 81)
        kernel = tt.load("gguf_linear", encoding=encoding, out_dtype="float32")
        xt = torch.from_numpy(x).cuda()
        buf = torch.empty(raw.nbytes + 2, dtype=torch.uint8, device=xt.device)
        shifted = buf[2:].view(raw.shape)
        shifted.copy_(torch.from_numpy(raw).cuda())
        assert shifted.data_ptr() % 4 == 2
        try:
            kernel(xt, shifted)
        except ValueError as error:
            assert "alignment" in str(error), error
        else:
            raise AssertionError(f"{encoding}: a 2-byte-aligned weight pointer was accepted")


def expect(oracle, got, x, raw, code, n, k):
    expected = oracle.linear(x, raw, code, n, k, prefill=x.shape[0] > 8)
    error = R.relative_l2(got.float().cpu().numpy(), expected)
    assert error <= TOLERANCE, error


def check_stream_order(kernel, xt, wt, reference):
    """Inputs written on a side stream just before the call: the launch must follow them there."""
    step("launch on a non-default torch stream")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        x = torch.empty_like(xt)
        x.copy_(xt)
        w = wt.clone()
        out = kernel(x, w)
        got = out.cpu()  # ordered after the kernel on the same stream
    assert torch.equal(got, reference.cpu())
    torch.cuda.synchronize()


def check_raw_into_prepare(kernel, xt, wt, reference):
    step("raw, into and prepare")
    assert torch.equal(kernel.raw(xt, wt).cpu(), reference.cpu())
    out = torch.full_like(reference, float("nan"))
    kernel.into(xt, wt, outputs=[out])
    assert torch.equal(out.cpu(), reference.cpu())
    x = xt.clone()
    prepared = kernel.prepare(x, wt)
    prepared()
    assert torch.equal(prepared.outputs[0].cpu(), reference.cpu())
    x.mul_(-1)  # in-place data changes are seen by the next submission
    prepared()
    negated = kernel.raw(x, wt)
    got = prepared.outputs[0]
    step(f"  negated input: max |prepared + reference| = {(got.float() + reference.float()).abs().max().item():.3g}")
    assert torch.equal(got.cpu(), negated.cpu())
    assert torch.linalg.norm(got.float() + reference.float()) <= TOLERANCE * torch.linalg.norm(reference.float())
    kernel(xt.clone(), wt)  # a launch through the cache leaves the prepared call's pointers alone
    prepared()
    assert torch.equal(prepared.outputs[0].cpu(), negated.cpu())
    x.set_(x.clone())
    try:
        prepared()
    except ValueError:
        pass
    else:
        raise AssertionError("a prepared call ran on changed storage")
    for bad in (xt.cpu(), xt[:, ::2]):
        try:
            kernel(bad, wt)
        except (TypeError, ValueError):
            pass
        else:
            raise AssertionError("a CPU or strided input was accepted")
    try:
        kernel.into(xt, wt, outputs=[torch.empty(reference.shape, dtype=torch.float32, device=xt.device)])
    except (ValueError, RuntimeError):
        pass
    else:
        raise AssertionError("an output of the wrong dtype was accepted")


def check_compile(oracle):
    step("torch.compile (aot_eager, dynamic shapes) over the registered operator")
    n, k = 512, 2048
    raw = cases.weight(n, k, "q4_k", 70)
    kernel = tt.load("gguf_linear", encoding="q4_k", out_dtype="float32")
    wt = torch.from_numpy(raw).cuda()

    def layer(x, w):
        return kernel(x, w) * 2.0 + 1.0

    compiled = torch.compile(layer, backend="aot_eager", dynamic=True, fullgraph=True)
    for m in (3, 5, 40):
        x = cases.activation(m, k, 71 + m)
        got = compiled(torch.from_numpy(x).cuda(), wt)
        expected = oracle.linear(x, raw, Q.Q4_K, n, k, prefill=m > 8) * 2.0 + 1.0
        error = R.relative_l2(got.cpu().numpy(), expected)
        assert error <= TOLERANCE, (m, error)


def check_bundle():
    step("hip bundle (derived scalar arguments) through torch")
    kernel = tt.load(str(ROOT / "tensor_amd" / "kernels" / "swiglu.tbin"))
    for _ in range(2):  # the second call of a shape takes the rebinding path (native plan or cached call)
        gate = torch.randn(7, 3001, dtype=torch.float16, device="cuda")
        up = torch.randn(7, 3001, dtype=torch.float16, device="cuda")
        out = kernel(gate, up)
        want = torch.nn.functional.silu(gate.float()) * up.float()
        assert torch.allclose(out.float(), want, rtol=2e-3, atol=2e-3)
    assert len(kernel._plans) == (1 if L.native_executor() else 0)


def check_overhead(kernel, xt, wt):
    step("host cost per call (not asserted)")
    prepared = kernel.prepare(xt, wt)
    for name, run in (("operator", lambda: kernel(xt, wt)), ("raw", lambda: kernel.raw(xt, wt)),
                      ("prepared", prepared)):
        for _ in range(20):
            run()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(500):
            run()
        torch.cuda.synchronize()
        step(f"  {name}: {(time.perf_counter() - start) / 500 * 1e6:.1f} us per call")


def check_import(session):
    step("Device.from_dlpack on a torch tensor: zero copy, producer held until release")
    source = torch.arange(1, 4097, dtype=torch.float32, device="cuda").reshape(64, 64)
    buffer = session.from_dlpack(source)
    assert buffer.pointer == source.data_ptr() and buffer.shape == (64, 64)
    source.mul_(3)
    assert np.array_equal(buffer.to_numpy(), source.cpu().numpy())
    buffer.release()
    step("Device.from_dlpack on a CPU tensor copies")
    host = torch.arange(10, dtype=torch.int32)
    copied = session.from_dlpack(host)
    assert np.array_equal(copied.to_numpy(), host.numpy())
    copied.release()


def check_export(session):
    step("torch.from_dlpack on a tensor_amd buffer: shared memory, release waits for torch")
    host = (np.arange(4096) % 1024).astype(np.float16).reshape(16, 256)  # x + 1 stays exact in fp16
    buffer = session.from_numpy(host)
    view = torch.from_dlpack(buffer)
    assert view.data_ptr() == buffer.pointer and view.shape == (16, 256) and view.dtype == torch.float16
    assert view.device.type == "cuda"
    view.add_(1)
    torch.cuda.synchronize()
    assert np.array_equal(buffer.to_numpy(), host + np.float16(1))
    try:
        buffer.release()
    except TensorRuntimeError:
        pass
    else:
        raise AssertionError("a buffer torch still views was released")
    del view
    gc.collect()
    buffer.release()


def check_showcase_call(oracle):
    """The showcase's GGUF case as benchmark.py runs it, with only the provider changed: a
    provider session on a torch stream (benchmark.py:840-844), torch tensors
    [x fp32 (M*K,), raw W bytes, out fp32 (M*N,)] (:453-464) imported with from_dlpack and
    launched by a TensorCall-style list of kernels (:276-290) on an executable specialised on
    (m, n, k), qualified by torch graph capture and replay after the input changes, with
    NaN-filled outputs (:499-555)."""
    import tensor_amd as tx

    stream = torch.cuda.Stream()
    with torch.inference_mode(), torch.cuda.stream(stream), \
            tx.Device(provider="hip", stream=stream.cuda_stream) as device:
        for encoding in (2, 12, 14):
            for m in (1, 32):
                n = k = 1024
                step(f"showcase packed call encoding={encoding} M={m}")
                raw = cases.weight(n, k, encoding, 600 + m).reshape(-1)
                inputs = [torch.randn(m * k, device="cuda", dtype=torch.float32) * 0.2, torch.from_numpy(raw).cuda()]
                out = torch.empty(m * n, device="cuda", dtype=torch.float32)
                kernels = [device.load("gguf_linear", encoding=encoding, m=m, n=n, k=k)]
                buffers = [[device.from_dlpack(t) for t in [*inputs, out]]]

                def call():
                    for kernel, args in zip(kernels, buffers):
                        kernel.launch(*args)

                call()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=torch.cuda.current_stream()):
                    call()
                saved = inputs[0].clone()
                for family in ("random", "fresh_scaled", "zero"):
                    if family == "fresh_scaled":
                        inputs[0].copy_(saved * -1.5)
                    elif family == "zero":
                        inputs[0].zero_()
                    out.fill_(float("nan"))
                    graph.replay()
                    torch.cuda.synchronize()
                    got = out.cpu().numpy()
                    x = inputs[0].cpu().numpy().reshape(m, k)
                    want = oracle.linear(x, raw, encoding, n, k, prefill=m > 1).reshape(-1)
                    assert not np.isnan(got).any(), family
                    error = R.relative_l2(got, want)
                    assert error <= (1e-5 if m == 1 else TOLERANCE), (encoding, m, family, error)
                del graph
                for args in buffers:
                    for buffer in args:
                        buffer.release()
                for kernel in kernels:
                    kernel.release()


def main():
    assert torch.cuda.is_available()
    step(f"torch {torch.__version__} hip {torch.version.hip}")
    executor = L.native_executor()
    step(f"native executor: {executor.__name__ if executor else None}")
    assert (executor is not None) == (os.environ.get("TENSOR_AMD_TORCH_NATIVE", "1") != "0")
    oracle = R.c_oracle()
    oracle.set_threads(16)
    kernel, xt, wt, out = check_linear(oracle, "q4_k", 1, 4096, 4096, "float16")
    assert len(tt.hip_runtimes()) == 1, tt.hip_runtimes()
    check_stream_order(kernel, xt, wt, out)
    check_raw_into_prepare(kernel, xt, wt, out)
    check_linear(oracle, "q4_k", 64, 1024, 4096, "float16")
    check_linear(oracle, "q6_k", 3, 1000, 2560, "float32")
    check_misaligned_weights()
    check_compile(oracle)
    check_bundle()
    check_showcase_call(oracle)
    session = S.session(torch.cuda.current_device())
    check_import(session)
    check_export(session)
    check_overhead(kernel, xt, wt)
    step("close, then launch again in a new session")
    tt.close()
    assert torch.equal(kernel(xt, wt).cpu(), out.cpu())
    tt.close()
    step("ok")


if __name__ == "__main__":
    main()
