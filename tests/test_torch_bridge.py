"""tensor_amd.torch host logic on the CPU: manifests, output metadata, the registered
operator's fake implementation and argument checks (no kernel runs here).

Fake ROCm tensors (torch's FakeTensorMode) stand in for device tensors, which
is also how torch.compile traces the operator.  Mirrors the reference's
tensor-torch contract (packages/tensor-torch/src/tensor_torch/kernel.py,
signatures.py, registration.py).
"""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

from torch._subclasses.fake_tensor import FakeTensorMode  # noqa: E402

import tensor_amd.torch as tt  # noqa: E402
from tensor_amd.gguf import quant as Q  # noqa: E402
from tensor_amd.gguf.kernels import manifest  # noqa: E402
from tensor_amd.torch import session as S  # noqa: E402

BUNDLE = "tensor_amd/kernels/swiglu.tbin"


def row_bytes(encoding, k):
    qk, block = Q.GEOMETRY[Q.ggml_type(encoding)]
    return k // qk * block


def fake(*shape, dtype=torch.float16):
    return torch.empty(*shape, dtype=dtype, device="cuda")


@pytest.mark.parametrize("encoding", ["q4_k", "q6_k", "q8_0", "q4_0"])
@pytest.mark.parametrize("out_dtype", ["float16", "float32"])
def test_linear_output_metadata(encoding, out_dtype):
    kernel = tt.Kernel("gguf_linear", encoding=encoding, out_dtype=out_dtype)
    assert [d["name"] for d in kernel.inputs] == ["x", "w"] and [d["name"] for d in kernel.outputs] == ["out"]
    with FakeTensorMode():
        x, w = fake(5, 512), fake(77, row_bytes(encoding, 512), dtype=torch.uint8)
        for symbolic in (False, True):
            assert kernel.metadata((x, w), symbolic=symbolic) == (
                [((5, 77), getattr(torch, out_dtype))], torch.device("cuda", 0))


def test_registered_operator_runs_its_fake_implementation():
    kernel = tt.load("gguf_linear", encoding="q4_k", out_dtype="float16")
    assert kernel.register() is kernel._op  # registered once
    with FakeTensorMode():
        out = kernel(fake(3, 1024), fake(40, row_bytes("q4_k", 1024), dtype=torch.uint8))
        assert out.shape == (3, 40) and out.dtype == torch.float16 and out.device.type == "cuda"
        outputs = [fake(3, 40)]
        kernel.into(fake(3, 1024), fake(40, row_bytes("q4_k", 1024), dtype=torch.uint8), outputs=outputs)
        with pytest.raises(Exception, match="metadata"):
            kernel.into(fake(3, 1024), fake(40, row_bytes("q4_k", 1024), dtype=torch.uint8),
                        outputs=[fake(3, 40, dtype=torch.float32)])


def test_swiglu_and_grouped_kernels():
    swiglu = tt.load("gguf_gemv_swiglu", encoding="q4_k")
    group = tt.load("gguf_gemv_group", encoding="q6_k", out_dtype="float32", count=3)
    assert [d["name"] for d in group.outputs] == ["out0", "out1", "out2"]
    with FakeTensorMode():
        x = fake(2, 512)
        w = fake(64, row_bytes("q4_k", 512), dtype=torch.uint8)
        assert swiglu(x, w, w).shape == (2, 64)
        rows = [fake(n, row_bytes("q6_k", 512), dtype=torch.uint8) for n in (8, 16, 24)]
        outs = group(x, *rows)
        assert [tuple(o.shape) for o in outs] == [(2, 8), (2, 16), (2, 24)]
        assert all(o.dtype == torch.float32 for o in outs)


def test_symbolic_checks_follow_the_manifest():
    gemv = tt.load("gguf_gemv", encoding="q4_k", out_dtype="float16")
    with FakeTensorMode():
        w = fake(16, row_bytes("q4_k", 512), dtype=torch.uint8)
        assert gemv(fake(8, 512), w).shape == (8, 16)
        with pytest.raises(RuntimeError, match="M is above 8"):
            gemv(fake(9, 512), w)
        with pytest.raises(RuntimeError, match="shape mismatch"):
            gemv(fake(1, 768), w)  # K = 768 needs 3 blocks per row
        with pytest.raises(ValueError, match="rank or dtype"):
            gemv(fake(1, 512, dtype=torch.float32), w)


def test_concrete_metadata_refuses_what_the_binder_refuses():
    kernel = tt.Kernel("gguf_linear", encoding="q4_0")
    with FakeTensorMode():
        w = fake(16, row_bytes("q4_0", 512), dtype=torch.uint8)
        with pytest.raises(ValueError):
            kernel.metadata((fake(2, 480), w))  # K not a multiple of 32 blocks' row
        with pytest.raises(ValueError, match="contiguous"):
            kernel.metadata((fake(512, 2).t(), w))
        with pytest.raises(ValueError, match="expected 2 inputs"):
            kernel.metadata((w,))
    with pytest.raises(TypeError, match="PyTorch tensor"):
        kernel.metadata(([1.0], w))
    with pytest.raises(ValueError, match="ROCm device"):
        kernel.metadata((torch.zeros(2, 512, dtype=torch.float16), torch.zeros(16, 288, dtype=torch.uint8)))


def test_bundle_kernel_with_derived_scalars():
    kernel = tt.Kernel(BUNDLE)
    assert [d["name"] for d in kernel.inputs] == ["gate", "up"]
    assert [s[1]["name"] for s in kernel._slots] == ["gate", "up", "out", "M", "N"]
    with FakeTensorMode():
        assert kernel.metadata((fake(4, 100), fake(4, 100)), symbolic=True)[0] == [((4, 100), torch.float16)]


def test_kernel_construction_checks():
    with pytest.raises(ValueError, match="module references"):
        tt.load("pkg::export")
    with pytest.raises(ValueError, match="options apply"):
        tt.Kernel(manifest("gguf_linear", "q4_k"), encoding="q4_k")
    with pytest.raises(ValueError, match="options apply"):
        tt.Kernel(BUNDLE, encoding="q4_k")
    with pytest.raises(ValueError, match="HIP provider"):
        tt.Kernel(dict(manifest("gguf_linear", "q4_k"), provider="cuda"))
    with pytest.raises(ValueError, match="mutable_inputs"):
        tt.Kernel("gguf_linear", encoding="q4_k", mutable_inputs=("out",))
    with pytest.raises(ValueError, match="declared outputs"):
        tt.Kernel(dict(manifest("gguf_linear", "q4_k"), outputs=[]))
    mutable = tt.Kernel(dict(manifest("gguf_linear", "q4_k"), outputs=[]), mutable_inputs=("x",))
    with pytest.raises(ValueError, match="mutable inputs"):
        mutable.register()


def test_each_load_is_its_own_operator():
    a, b = tt.load("gguf_linear", encoding="q8_0"), tt.load("gguf_linear", encoding="q8_0")
    assert a._op is not b._op and a._op._name != b._op._name


def test_two_hip_runtimes_are_refused(monkeypatch):
    assert isinstance(S.hip_runtimes(), set)
    monkeypatch.setattr(S, "hip_runtimes", lambda: {"/opt/rocm/lib/libamdhip64.so.7", "/torch/lib/libamdhip64.so"})
    with pytest.raises(RuntimeError, match="two HIP runtimes"):
        S._check_single_runtime()
    monkeypatch.setattr(S, "hip_runtimes", lambda: {"/torch/lib/libamdhip64.so"})
    S._check_single_runtime()
