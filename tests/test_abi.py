"""C-ABI contract of libtensor_hip.so, checked on the CPU.

Mirrors the reference's descriptor-tampering tests
(tests/runtime/test_runtime_abi.py:33-44, :89-104; src/tensor/native/host.cpp:78-83):
every malformed call is rejected with the right status before any device
state is touched, so none of these calls needs a GPU.
"""

from __future__ import annotations

import ctypes as c
import re
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

from tensor_amd import _native
from tensor_amd.gguf import kernels
from tensor_amd.runtime import abi
from tensor_amd.runtime.signature import Signature, bind_shapes

ROOT = Path(__file__).resolve().parents[1]
OK, ERR_ABI, ERR_ARG, ERR_PROVIDER = 0, 1, 2, 3


def test_descriptor_sizes():
    assert [c.sizeof(s) for s in (abi.BufferDescriptor, abi.Argument, abi.StreamDescriptor,
                                  abi.CallDescriptor, abi.ErrorDescriptor, abi.WorkspaceRequirements,
                                  abi.ExecutableDescriptor, abi.EventDescriptor)] == [48, 64, 16, 72, 512, 24, 64, 40]


def declared_functions():
    names = []
    for header in sorted((ROOT / "include").rglob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:int32_t|const char\s*\*)\s*\*?\s*(\w+)\s*\(", text, flags=re.M)
    return names


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    names = declared_functions()
    assert "tensor_gguf_gemv_v1" in names and "tensor_hip_malloc" in names
    missing = [name for name in names if not hasattr(lib, name)]
    assert not missing, missing
    assert set(_native.KERNELS) | set(_native.SERVICES) | {"tensor_hip_version", "tensor_hip_source_hash",
                                                          "tensor_hip_module_launch_v1"} == set(names)


class Call:
    """A well-formed 4-argument linear call with fake (never dereferenced) addresses."""

    def __init__(self, m=1, n=64, k=512, type_=12, out_dtype=10, block=144, qk=256):
        self.shapes = [(m, k), (n, k // qk * block), (m, n)]
        dtypes = [10, 3, out_dtype]
        items = [2, 1, 2 if out_dtype == 10 else 4]
        self.keep = []
        self.args = (abi.Argument * 4)()
        for i, (shape, dtype, item) in enumerate(zip(self.shapes, dtypes, items)):
            shp = (c.c_int64 * 2)(*shape)
            strides = (c.c_int64 * 2)(shape[1] * item, item)
            self.keep += [shp, strides]
            self.args[i].kind = 1
            self.args[i].dtype = dtype
            self.args[i].buffer = abi.BufferDescriptor(0x10000 * (i + 1), shape[0] * shape[1] * item, shp, strides,
                                                       2, dtype, 10, 0)
        self.args[3].kind = 2
        self.args[3].dtype = 7
        self.args[3].scalar = type_
        self.call = abi.CallDescriptor(1, 72, self.args, 4, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self, entry="tensor_gguf_gemv_v1"):
        error = abi.ErrorDescriptor()
        error.message = b"x" * 507
        status = _native.kernel(entry)(c.byref(self.call), c.byref(error))
        return status, error.message.decode()


def tamper(**changes):
    call = Call(**changes.pop("shape", {}))
    for path, value in changes.items():
        target = call
        parts = path.split(".")
        for part in parts[:-1]:
            target = target[int(part)] if part.isdigit() else getattr(target, part)
        setattr(target, parts[-1], value)
    return call


@pytest.mark.parametrize("mutation,code,needle", [
    ({"call.abi_version": 2}, ERR_ABI, "ABI"),
    ({"call.struct_size": 8}, ERR_ABI, "ABI"),
    ({"call.flags": 1}, ERR_ARG, "argument count or flags"),
    ({"call.argument_count": 3}, ERR_ARG, "argument count or flags"),
    ({"call.stream.device_type": 1}, ERR_PROVIDER, "ROCm stream"),
    ({"args.3.scalar": 5}, ERR_ARG, "unsupported GGML type"),
    ({"args.3.scalar": (1 << 32) | 12}, ERR_ARG, "noncanonical"),
    ({"args.3.kind": 1}, ERR_ARG, "type: wrong argument kind"),
    ({"args.0.dtype": 11}, ERR_ARG, "x: wrong argument kind or dtype"),
    ({"args.0.buffer.byte_size": 4}, ERR_ARG, "x: insufficient buffer storage"),
    ({"args.0.buffer.address": 0x10008}, ERR_ARG, "x: invalid buffer descriptor"),
    ({"args.1.buffer.device_type": 2}, ERR_ARG, "w: invalid buffer descriptor"),
    ({"args.1.buffer.device_ordinal": 1}, ERR_ARG, "w: invalid buffer descriptor"),
    ({"args.2.buffer.rank": 3}, ERR_ARG, "out: invalid buffer descriptor"),
    ({"args.2.kind": 2}, ERR_ARG, "out: wrong argument kind"),
])
def test_malformed_calls_are_rejected(mutation, code, needle):
    status, message = tamper(**mutation).run()
    assert status == code, message
    assert needle in message
    assert len(message) < 507  # NUL-terminated, overwritten


def test_stride_and_shape_mismatches():
    call = Call()
    call.keep[1][1] = 8  # x element stride of 8 bytes
    assert call.run() == (ERR_ARG, "x: shape, stride or size mismatch")
    call = Call(n=64, k=512)
    call.keep[2][1] = 144 * 3  # w rows hold 3 super-blocks but K needs 2
    call.args[1].buffer.byte_size = 64 * 144 * 3
    call.keep[3][0] = 144 * 3
    assert call.run()[0] == ERR_ARG
    call = Call(m=2, n=64)
    call.keep[4][0] = 3  # out rows != M
    call.args[2].buffer.byte_size = 3 * 64 * 2
    assert call.run() == (ERR_ARG, "out: shape, stride or size mismatch")


def test_k_must_be_whole_blocks():
    call = Call(k=512)
    call.keep[0][1] = 300
    call.keep[1][0] = 600
    call.args[0].buffer.byte_size = 600
    assert call.run()[0] == ERR_ARG


def test_gemv_row_limit_but_gemm_accepts():
    status, message = Call(m=9).run("tensor_gguf_gemv_v1")
    assert status == ERR_ARG and "at most 8" in message


def test_null_call():
    error = abi.ErrorDescriptor()
    assert _native.kernel("tensor_gguf_gemv_v1")(None, c.byref(error)) == ERR_ABI
    assert _native.kernel("tensor_gguf_dequant_v1")(None, None) == ERR_ABI


def test_dequant_argument_checks():
    call = Call()
    args = (abi.Argument * 3)(call.args[1], call.args[2], call.args[3])
    call.call.arguments = args
    call.call.argument_count = 3
    # out [1, 64] does not match w [64, 288] -> rejected
    status, message = call.run("tensor_gguf_dequant_v1")
    assert status == ERR_ARG and "out" in message


class GroupCall:
    """A well-formed grouped GEMV call [x, (w_i, out_i)..., type] with fake addresses."""

    def __init__(self, rows=(64, 32), m=1, k=512, type_=12, block=144, qk=256):
        count = len(rows)
        shapes = [(m, k)]
        dtypes, items = [10], [2]
        for n in rows:
            shapes += [(n, k // qk * block), (m, n)]
            dtypes += [3, 10]
            items += [1, 2]
        self.keep = []
        self.args = (abi.Argument * (2 * count + 2))()
        for i, (shape, dtype, item) in enumerate(zip(shapes, dtypes, items)):
            shp = (c.c_int64 * 2)(*shape)
            strides = (c.c_int64 * 2)(shape[1] * item, item)
            self.keep += [shp, strides]
            self.args[i].kind = 1
            self.args[i].dtype = dtype
            self.args[i].buffer = abi.BufferDescriptor(0x10000 * (i + 1), shape[0] * shape[1] * item, shp, strides,
                                                       2, dtype, 10, 0)
        last = 2 * count + 1
        self.args[last].kind = 2
        self.args[last].dtype = 7
        self.args[last].scalar = type_
        self.call = abi.CallDescriptor(1, 72, self.args, 2 * count + 2, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self):
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_gemv_group_v1")(c.byref(self.call), c.byref(error))
        return status, error.message.decode()


def test_group_call_argument_checks():
    call = GroupCall(rows=(64, 32, 16))
    call.call.argument_count = 7  # odd: not [x, pairs..., type]
    assert call.run() == (ERR_ARG, "invalid argument count or flags")
    call = GroupCall(rows=(64, 32))
    call.call.argument_count = 10  # beyond three matrices
    assert call.run()[0] == ERR_ARG
    call = GroupCall(rows=(64, 32))
    call.keep[8][1] = 31  # out1 columns != N1 (a consistent [1, 31] descriptor)
    call.keep[9][0] = 31 * 2
    call.args[4].buffer.byte_size = 31 * 2
    assert call.run() == (ERR_ARG, "out1: shape, stride, size or dtype mismatch")
    call = GroupCall(rows=(64, 32), m=9)
    status, message = call.run()
    assert status == ERR_ARG and "at most 8" in message
    call = GroupCall(rows=(64,))
    call.args[3].scalar = 5
    status, message = call.run()
    assert status == ERR_ARG and "unsupported GGML type" in message


def test_group_manifest_binds_each_matrix():
    manifest = kernels.manifest("gguf_gemv_group", "q4_k", "float16", count=3)
    assert manifest["outputs"] == ["out0", "out1", "out2"]
    k = 4096
    buffers = {"x": fake((1, k), "float16")}
    for i, n in enumerate((4096, 1024, 1024)):
        buffers[f"w{i}"] = fake((n, k // 256 * 144), "uint8")
        buffers[f"out{i}"] = fake((1, n), "float16")
    symbols, _ = bind_shapes(manifest, buffers)
    assert symbols == {"M": 1, "K": 4096, "N0": 4096, "N1": 1024, "N2": 1024}
    with pytest.raises(ValueError):
        kernels.manifest("gguf_gemv_group", "q4_k", count=4)
    with pytest.raises(ValueError):
        kernels.manifest("gguf_gemv", "q4_k", count=2)


class SwigluCall:
    """A well-formed SwiGLU GEMV call [x, w_gate, w_up, out, type] with fake addresses."""

    def __init__(self, m=1, n=64, k=512, type_=12, block=144, qk=256, up_rows=None):
        shapes = [(m, k), (n, k // qk * block), (up_rows or n, k // qk * block), (m, n)]
        dtypes, items = [10, 3, 3, 10], [2, 1, 1, 2]
        self.keep = []
        self.args = (abi.Argument * 5)()
        for i, (shape, dtype, item) in enumerate(zip(shapes, dtypes, items)):
            shp = (c.c_int64 * 2)(*shape)
            strides = (c.c_int64 * 2)(shape[1] * item, item)
            self.keep += [shp, strides]
            self.args[i].kind = 1
            self.args[i].dtype = dtype
            self.args[i].buffer = abi.BufferDescriptor(0x10000 * (i + 1), shape[0] * shape[1] * item, shp, strides,
                                                       2, dtype, 10, 0)
        self.args[4].kind = 2
        self.args[4].dtype = 7
        self.args[4].scalar = type_
        self.call = abi.CallDescriptor(1, 72, self.args, 5, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self):
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_gemv_swiglu_v1")(c.byref(self.call), c.byref(error))
        return status, error.message.decode()


def test_swiglu_call_argument_checks():
    call = SwigluCall()
    call.call.argument_count = 4
    assert call.run() == (ERR_ARG, "invalid argument count or flags")
    assert SwigluCall(up_rows=63).run() == (ERR_ARG, "w_up: shape differs from w_gate")
    call = SwigluCall()
    call.args[2].dtype = call.args[2].buffer.dtype = 10  # fp16 in place of raw bytes
    assert call.run() == (ERR_ARG, "w_up: wrong argument kind or dtype")
    status, message = SwigluCall(m=9).run()
    assert status == ERR_ARG and "at most 8" in message
    call = SwigluCall()
    call.keep[6][1] = 63  # out columns != N (a consistent [1, 63] descriptor)
    call.keep[7][0] = 63 * 2
    call.args[3].buffer.byte_size = 63 * 2
    assert call.run() == (ERR_ARG, "out: shape, stride or size mismatch")
    status, message = SwigluCall(type_=5).run()
    assert status == ERR_ARG and "unsupported GGML type" in message
    # a Q8_0 pair whose rows are not whole blocks
    status, message = SwigluCall(k=40, type_=8, block=34, qk=32).run()
    assert status == ERR_ARG and "w_gate" in message


def test_swiglu_manifest_binds_gate_and_up():
    manifest = kernels.manifest("gguf_gemv_swiglu", "q4_k", "float16")
    assert manifest["entrypoint"] == "tensor_gguf_gemv_swiglu_v1" and manifest["outputs"] == ["out"]
    assert [a["name"] for a in manifest["arguments"]] == ["x", "w_gate", "w_up", "out", "type"]
    k, n = 4096, 12288
    buffers = {"x": fake((1, k), "float16"), "w_gate": fake((n, k // 256 * 144), "uint8"),
               "w_up": fake((n, k // 256 * 144), "uint8"), "out": fake((1, n), "float16")}
    symbols, _ = bind_shapes(manifest, buffers)
    assert symbols == {"M": 1, "N": n, "K": k}
    with pytest.raises(ValueError):
        bind_shapes(manifest, dict(buffers, w_up=fake((n - 16, k // 256 * 144), "uint8")))
    with pytest.raises(ValueError, match="outside"):
        bind_shapes(manifest, dict(buffers, x=fake((9, k), "float16"), out=fake((9, n), "float16")))


# --------------------------------------------------------- manifest binding --

def fake(shape, dtype):
    return SimpleNamespace(shape=tuple(shape), dtype=np.dtype(dtype))


@pytest.mark.parametrize("encoding,qk,block", [("q4_k", 256, 144), ("q6_k", 256, 210), ("q8_0", 32, 34), ("q4_0", 32, 18)])
def test_manifest_binds_gguf_shapes(encoding, qk, block):
    manifest = kernels.manifest("gguf_linear", encoding)
    x, w, out = fake((4, 4096), "float16"), fake((128, 4096 // qk * block), "uint8"), fake((4, 128), "float16")
    symbols, values = bind_shapes(manifest, {"x": x, "w": w, "out": out})
    assert symbols == {"M": 4, "K": 4096, "N": 128}
    with pytest.raises(ValueError):
        bind_shapes(manifest, {"x": x, "w": fake((128, 4096 // qk * block + block), "uint8"), "out": out})
    with pytest.raises(ValueError):
        bind_shapes(manifest, {"x": fake((4, qk + qk // 2), "float16"), "w": fake((128, block), "uint8"),
                               "out": out})
    assert manifest["constants"]["type"] == Q_TYPES[encoding]


Q_TYPES = {"q4_0": 2, "q8_0": 8, "q4_k": 12, "q6_k": 14}


def test_gemv_manifest_domain():
    manifest = kernels.manifest("gguf_gemv", "q4_k", out_dtype="float32")
    bind_shapes(manifest, {"x": fake((8, 256), "float16"), "w": fake((2, 144), "uint8"), "out": fake((8, 2), "float32")})
    with pytest.raises(ValueError, match="outside"):
        bind_shapes(manifest, {"x": fake((9, 256), "float16"), "w": fake((2, 144), "uint8"),
                               "out": fake((9, 2), "float32")})


def test_bound_call_carries_constant_type_scalar():
    manifest = kernels.manifest("gguf_linear", "q6_k")
    device = SimpleNamespace(stream_descriptor=lambda: abi.StreamDescriptor(10, 0, 0))
    buffers = {}
    for name, shape, dtype in (("x", (1, 256), "float16"), ("w", (3, 210), "uint8"), ("out", (1, 3), "float16")):
        b = SimpleNamespace(shape=shape, dtype=np.dtype(dtype))
        b._descriptor = abi.BufferDescriptor(0x1000, 0, None, None, 2, abi.DTYPES[dtype], 10, 0)
        buffers[name] = b
    symbols, values = bind_shapes(manifest, buffers)
    launch = {"grid": [1, 1, 1], "block": [256, 1, 1], "shared_memory_bytes": 0}
    executable = SimpleNamespace(signature=Signature(manifest), device=device)
    call = abi.BoundCall(executable, values, symbols, launch, device.stream_descriptor())
    assert [a.kind for a in call.arguments] == [1, 1, 1, 2]
    assert call.arguments[3].dtype == abi.DTYPES["uint32"] and call.arguments[3].scalar == 14
    assert call.descriptor.stream.device_type == 10


def test_unknown_kernel_and_encoding():
    with pytest.raises(ValueError):
        kernels.manifest("gguf_conv", "q4_k")
    with pytest.raises(ValueError):
        kernels.manifest("gguf_linear", "iq4_xs")
    with pytest.raises(ValueError):
        kernels.manifest("gguf_linear", 15)  # Q8_K: an intermediate format, not a weight encoding
    with pytest.raises(ValueError):
        kernels.manifest("gguf_linear", "q4_k", out_dtype="bfloat16")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_native.NativeLibraryError, match="not built"):
        _native.library(tmp_path / "libtensor_hip.so")


class PackedCall:
    """The showcase's packed call form (benchmark.py:460-464): flat fp32 x [M*K], flat raw w,
    flat fp32 out [M*N], then type, m, n, k scalars; fake (never dereferenced) addresses."""

    def __init__(self, m=1, n=1024, k=1024, type_=2, qk=32, block=18, w_dtype=3, w_item=1):
        sizes = [(m * k, 11, 4), (n * k // qk * block // w_item, w_dtype, w_item), (m * n, 11, 4)]
        self.keep = []
        self.args = (abi.Argument * 7)()
        for i, (count, dtype, item) in enumerate(sizes):
            shp = (c.c_int64 * 1)(count)
            strides = (c.c_int64 * 1)(item)
            self.keep += [shp, strides]
            self.args[i].kind = 1
            self.args[i].dtype = dtype
            self.args[i].buffer = abi.BufferDescriptor(0x100000 * (i + 1), count * item, shp, strides, 1, dtype, 10, 0)
        for i, value in enumerate((type_, m, n, k)):
            self.args[3 + i].kind = 2
            self.args[3 + i].dtype = 7
            self.args[3 + i].scalar = value
        self.call = abi.CallDescriptor(1, 72, self.args, 7, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self):
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_packed_v1")(c.byref(self.call), c.byref(error))
        return status, error.message.decode()


def packed(**changes):
    call = PackedCall(**changes.pop("shape", {}))
    for path, value in changes.items():
        target = call
        parts = path.split(".")
        for part in parts[:-1]:
            target = target[int(part)] if part.isdigit() else getattr(target, part)
        setattr(target, parts[-1], value)
    return call


@pytest.mark.parametrize("mutation,code,needle", [
    ({"call.abi_version": 2}, ERR_ABI, "ABI"),
    ({"call.struct_size": 8}, ERR_ABI, "ABI"),
    ({"call.argument_count": 4}, ERR_ARG, "argument count or flags"),
    ({"call.stream.device_type": 1}, ERR_PROVIDER, "ROCm stream"),
    ({"args.3.scalar": 9}, ERR_ARG, "unsupported GGML type"),
    ({"args.4.scalar": 0}, ERR_ARG, "m, n, k"),
    ({"args.6.scalar": 1000}, ERR_ARG, "m, n, k"),  # not a multiple of QK = 32
    ({"args.5.dtype": 6}, ERR_ARG, "n: wrong argument kind or dtype"),
    ({"args.0.dtype": 12}, ERR_ARG, "x: wrong argument kind or dtype"),
    ({"args.0.buffer.byte_size": 4}, ERR_ARG, "x: insufficient buffer storage"),
    ({"args.0.buffer.device_type": 1}, ERR_ARG, "x: invalid buffer descriptor"),
    ({"args.1.dtype": 11, "args.1.buffer.dtype": 11}, ERR_ARG, "w: wrong argument kind or dtype"),
    ({"args.2.buffer.rank": 0}, ERR_ARG, "out: invalid buffer descriptor"),
    ({"args.5.scalar": 1023}, ERR_ARG, "w: holds"),  # the shape no longer matches w's bytes
])
def test_packed_form_rejects_malformed_calls(mutation, code, needle):
    status, message = packed(**mutation).run()
    assert status == code, message
    assert needle in message, message


@pytest.mark.parametrize("shape", [{}, {"m": 32}, {"type_": 12, "qk": 256, "block": 144},
                                    {"type_": 14, "qk": 256, "block": 210, "w_dtype": 5, "w_item": 2}])
def test_packed_form_accepts_the_showcase_call(shape):
    """A well-formed call passes every descriptor check and reaches the device check (the
    CPU container has no HIP device, so the status is the provider's)."""
    status, message = PackedCall(**shape).run()
    assert status == ERR_PROVIDER, message
    assert "hipGetDevice" in message or "current device" in message, message


def test_gemm_workspace_query_follows_the_split_plan():
    """The grouped prefill GEMM splits K across workgroups only where its plan does, and says
    how many bytes of fp32 partial sums it then needs (splits x M x sum(N) x 4)."""
    query = lambda t, m, k, rows: _query_workspace(t, m, k, rows)
    assert query(12, 256, 4096, [4096, 1024, 1024]) == 4 * 256 * 6144 * 4   # C5 q + k + v
    assert query(14, 256, 12288, [4096]) == 8 * 256 * 4096 * 4             # C5 down (Q6_K)
    assert query(12, 256, 4096, [4096]) == 0                                # o: small tiles fill the CUs
    assert query(12, 2048, 4096, [12288]) == 0                              # C4: 256 x 128 tiles fill them
    assert query(12, 256, 4096, [12288, 12288]) == 0                        # gate + up
    assert query(8, 256, 12288, [4096]) == 8 * 256 * 4096 * 4             # Q8_0 down: pipelined too
    assert query(8, 256, 12320, [4096]) == 0                                # K % 64 == 32: generic tiles
    assert query(3, 256, 12288, [4096]) == 0                                # generic encodings never split
    assert query(12, 32, 4096, [4096, 1024, 1024]) == 2 * 32 * 6144 * 4    # q + k + v at M=32: 64 x 64, 2 splits
    assert query(12, 32, 1024, [1024]) == 0                                 # showcase M=32: the small-M kernel
    assert query(14, 128, 12288, [4096]) == 8 * 128 * 4096 * 4            # down at M=128: 256 x 128, 8 splits
    assert query(12, 128, 4096, [4096, 1024, 1024]) == 0                    # q + k + v at M=128: 64 x 64 tiles fill them


def _query_workspace(type_, m, k, rows):
    result = c.c_uint64()
    error = abi.ErrorDescriptor()
    status = _native.library().tensor_gguf_gemm_workspace_v1(type_, m, k, (c.c_int64 * len(rows))(*rows), len(rows),
                                                             c.byref(result), c.byref(error))
    assert status == OK, error.message
    return result.value


class GroupGemmCall:
    """[x, w0, out0, w1, out1, workspace, type] with fake (never dereferenced) addresses."""

    def __init__(self, m=256, k=512, rows=(64, 32), ws=4096):
        shapes = [((m, k), 10, 2)]
        for n in rows:
            shapes += [((n, k // 256 * 144), 3, 1), ((m, n), 10, 2)]
        self.keep, self.args = [], (abi.Argument * (len(shapes) + 2))()
        for i, (shape, dtype, item) in enumerate(shapes):
            shp, strides = (c.c_int64 * 2)(*shape), (c.c_int64 * 2)(shape[1] * item, item)
            self.keep += [shp, strides]
            self.args[i].kind, self.args[i].dtype = 1, dtype
            self.args[i].buffer = abi.BufferDescriptor(0x100000 * (i + 1), shape[0] * shape[1] * item, shp, strides,
                                                       2, dtype, 10, 0)
        wshape, wstride = (c.c_int64 * 1)(ws), (c.c_int64 * 1)(1)
        self.keep += [wshape, wstride]
        w = len(shapes)
        self.args[w].kind, self.args[w].dtype = 1, 3
        self.args[w].buffer = abi.BufferDescriptor(0x4000000, ws, wshape, wstride, 1, 3, 10, 0)
        self.args[w + 1].kind, self.args[w + 1].dtype, self.args[w + 1].scalar = 2, 7, 12
        self.call = abi.CallDescriptor(1, 72, self.args, len(shapes) + 2, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self, entry="tensor_gguf_gemm_group_v1"):
        error = abi.ErrorDescriptor()
        status = _native.kernel(entry)(c.byref(self.call), c.byref(error))
        return status, error.message.decode()


def test_gemm_group_call_argument_checks():
    call = GroupGemmCall()
    status, message = call.run()
    assert status == ERR_PROVIDER, message  # well formed: stops at the device check
    call = GroupGemmCall()
    call.args[5].dtype = call.args[5].buffer.dtype = 11
    assert call.run() == (ERR_ARG, "workspace: wrong argument kind or dtype")
    call = GroupGemmCall()
    call.args[5].buffer.address = 0x4000010  # not 256-byte aligned
    assert call.run() == (ERR_ARG, "workspace: invalid buffer descriptor")
    call = GroupGemmCall()
    call.call.argument_count = 6
    assert call.run()[0] == ERR_ARG
    call = GroupGemmCall()
    call.keep[8][0] = 255  # out1 with 255 rows for M = 256
    assert call.run() == (ERR_ARG, "out1: shape, stride, size or dtype mismatch")


def test_gemm_group_noalloc_takes_the_group_without_a_workspace():
    noalloc = "tensor_gguf_gemm_group_noalloc_v1"
    call = GroupGemmCall()
    assert call.run(noalloc) == (ERR_ARG, "invalid argument count or flags")  # a workspace is one too many
    call = GroupGemmCall()
    call.args[5] = call.args[6]  # [x, w0, out0, w1, out1, type]
    call.call.argument_count = 6
    status, message = call.run(noalloc)
    assert status == ERR_PROVIDER, message  # well formed: stops at the device check
    call.keep[8][0] = 255
    assert call.run(noalloc) == (ERR_ARG, "out1: shape, stride, size or dtype mismatch")
    call.call.argument_count = 5
    assert call.run(noalloc)[0] == ERR_ARG


def test_gemm_plan_query_names_the_library_plans_at_the_baseline_shapes():
    """The plans the grouped prefill GEMM takes at C4 and C5 (CPU only: a query, no launch)."""
    from tensor_amd.providers.hip import gemm_tiles

    tiles = gemm_tiles()
    assert tiles[0] == {"bm": 256, "bn": 128, "ks": 1} and tiles[8] == {"bm": 256, "bn": 96, "ks": 1}
    assert tiles[9] == {"bm": 256, "bn": 192, "ks": 1}
    lib = _native.library()

    def plan(code, m, k, rows, workspace=1 << 30):
        tile, splits, pipelined = c.c_int32(), c.c_int32(), c.c_int32()
        error = abi.ErrorDescriptor()
        status = lib.tensor_gguf_gemm_plan_v1(code, m, k, (c.c_int64 * len(rows))(*rows), len(rows), workspace,
                                              c.byref(tile), c.byref(splits), c.byref(pipelined), c.byref(error))
        assert status == OK, error.message
        return tile.value, splits.value, bool(pipelined.value)

    assert plan(12, 512, 4096, [12288]) == (8, 1, True)            # C4 M=512: 256 x 96, one round
    assert plan(12, 2048, 4096, [12288]) == (9, 1, True)           # C4 M=2048: 256 x 192, x by LDS DMA
    assert plan(12, 1536, 4096, [12288]) == (9, 1, True)           # two rounds of 256 x 192 against three
    assert plan(12, 256, 4096, [4096, 1024, 1024]) == (0, 4, True)  # C5 q + k + v, K split 4 ways
    assert plan(12, 256, 4096, [4096]) == (7, 1, True)             # C5 o: 64 x 64, K over 4 wave groups
    assert plan(12, 256, 4096, [12288, 12288]) == (8, 1, True)     # C5 gate + up
    assert plan(14, 256, 12288, [4096]) == (0, 8, True)            # C5 down (Q6_K), K split 8 ways
    assert plan(14, 256, 12288, [4096], workspace=0) == (7, 1, True)  # no workspace: no split
    # the pipelined kernels address a matrix by 32-bit offsets: 4 GiB and up takes the generic one
    assert plan(12, 256, 4096, [1_800_000])[2] is True               # 3.86 GiB
    assert plan(12, 256, 4096, [1_900_000])[2] is False              # 4.08 GiB
    error = abi.ErrorDescriptor()
    assert lib.tensor_gguf_gemm_tile_v1(len(tiles), c.byref(c.c_int32()), c.byref(c.c_int32()),
                                        c.byref(c.c_int32()), c.byref(error)) == ERR_ARG


def test_gemv_plan_query_names_the_library_plans_at_the_baseline_shapes():
    """The multi-row plans the Q4_K decode GEMV takes at C2's M=4 and M=8 shapes (CPU only: a
    query, no launch), and the paths the query leaves to other kernels."""
    from tensor_amd.providers.hip import GEMV_FIELDS, GEMV_KERNELS

    assert GEMV_KERNELS == ("sec", "mt", "mfma", "sec_split")
    lib = _native.library()

    def plan(code, m, k, n):
        kernel, a, b = c.c_int32(), c.c_int32(), c.c_int32()
        error = abi.ErrorDescriptor()
        status = lib.tensor_gguf_gemv_plan_v1(code, m, k, n, c.byref(kernel), c.byref(a), c.byref(b), c.byref(error))
        assert status == OK, error.message
        return kernel.value, a.value, b.value

    assert plan(12, 4, 4096, 12288) == (0, 3, 1)   # gate / up at M=4: sector tiles, 3 per workgroup, x first
    assert plan(12, 4, 12288, 4096) == (0, 1, 0)   # down at M=4: one tile, 12 K ranges, 96 KB of x
    #                                                staged behind the weight loads
    assert plan(12, 8, 4096, 12288) == (0, 3, 0)   # gate at M=8: 64 KB of x, behind the weight loads
    assert plan(12, 8, 12288, 4096) == (3, 4, 4)   # down at M=8: x (196 KB) does not fit LDS, so K splits
    #                                                into 4 ranges, 4 tiles per workgroup: 256 workgroups
    assert plan(12, 8, 12288, 64) == (2, 8, 0)     # too few tiles for a split round: x read per wave
    assert plan(12, 4, 4096, 4096) == (1, 1, 2)    # narrower shapes: the multi-tile kernel
    for query in ((12, 1, 4096, 12288), (14, 4, 4096, 4096), (8, 4, 4096, 4096)):
        assert plan(*query)[0] == -1               # M = 1 and the other encodings: other kernels
    for kernel, a, b in (plan(12, 4, 4096, 12288), plan(12, 8, 12288, 4096), plan(12, 4, 4096, 4096)):
        assert (a, b) in GEMV_FIELDS[kernel]
    error = abi.ErrorDescriptor()
    out = [c.c_int32() for _ in range(3)]
    assert lib.tensor_gguf_gemv_plan_v1(12, 9, 4096, 4096, *map(c.byref, out), c.byref(error)) == ERR_ARG
    assert lib.tensor_gguf_gemv_plan_v1(12, 4, 4000, 4096, *map(c.byref, out), c.byref(error)) == ERR_ARG


def test_gemv_k_split_plans_stay_in_one_round_and_fit_the_scratch():
    """Where the multi-row plan splits K across workgroups (kernel 3), its workgroups make one
    round on 256 CUs (128-256 of them), each K range is whole 1024-column sectors, and the fp32
    partial sums fit the library's 32 MiB scratch; shapes whose x fits in LDS never split."""
    lib = _native.library()

    def plan(m, k, n):
        kernel, a, b = c.c_int32(), c.c_int32(), c.c_int32()
        error = abi.ErrorDescriptor()
        assert lib.tensor_gguf_gemv_plan_v1(12, m, k, n, c.byref(kernel), c.byref(a), c.byref(b),
                                            c.byref(error)) == OK, error.message
        return kernel.value, a.value, b.value

    seen = 0
    for m in range(2, 9):
        for k in (4096, 8192, 12288, 16384):
            for n in (64, 300, 1000, 2048, 4096, 4100, 8192, 12288):
                kernel, per, splits = plan(m, k, n)
                if kernel != 3:
                    continue
                seen += 1
                tiles = (n + 15) // 16
                grid = -(-tiles // per) * splits
                assert m >= 4 and splits in (2, 4), (m, k, n, per, splits)
                assert 128 <= grid <= 256, (m, k, n, per, splits, grid)
                assert k % (1024 * splits) == 0 and per * (k // 1024 // splits) <= 16
                assert splits * m * n * 4 <= 32 << 20
                assert m * k * 2 > 64 * 1024, (m, k)  # x of the whole row would not fit with its tables
    assert seen >= 10
    assert plan(8, 12288, 4096) == (3, 4, 4)


def test_gemv_variant_refuses_a_plan_that_does_not_fit():
    """tensor_gguf_gemv_variant_v1 checks the named kernel and fields against the shape before
    any HIP call (fake device addresses; CPU only): a plan that fits gets as far as the device
    check, which fails here with no GPU."""
    manifest = kernels.manifest("gguf_gemv_variant", "q4_k", "float16")
    names = [a["name"] for a in manifest["arguments"]]
    assert names == ["x", "w", "out", "type", "kernel", "a", "b"]
    with pytest.raises(ValueError):
        kernels.manifest("gguf_gemv_variant", "q6_k", "float16")

    def call_with(m, n, k, kernel, a, b, code=12):
        shapes = {"x": (m, k), "w": (n, k // 256 * 144), "out": (m, n)}
        dtypes, sizes = {"x": 10, "w": 3, "out": 10}, {"x": 2, "w": 1, "out": 2}
        keep, args = [], (abi.Argument * 7)()
        for j, name in enumerate(names[:3]):
            shape = shapes[name]
            strides = (sizes[name] * shape[1], sizes[name])
            arrays = ((c.c_int64 * 2)(*shape), (c.c_int64 * 2)(*strides))
            keep.append(arrays)
            args[j].kind, args[j].dtype = 1, dtypes[name]
            args[j].buffer = abi.BufferDescriptor(0x10000 * (j + 1), int(np.prod(shape)) * sizes[name], arrays[0],
                                                  arrays[1], 2, dtypes[name], 10, 0)
        for j, value in ((3, code), (4, kernel), (5, a), (6, b)):
            args[j].kind, args[j].dtype, args[j].scalar = 2, 7, value
        call = abi.CallDescriptor(1, 72, args, 7, 0, (c.c_uint32 * 3)(1, 1, 1), (c.c_uint32 * 3)(256, 1, 1), 0,
                                  abi.StreamDescriptor(10, 0, 0))
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_gemv_variant_v1")(c.byref(call), c.byref(error))
        return status, error.message.decode()

    assert call_with(4, 4096, 12288, 0, 3, 1)[0] == ERR_ARG    # 3 tiles x 12 K ranges > 16 waves
    assert call_with(8, 4096, 12288, 1, 1, 3)[0] == ERR_ARG    # x of 8 x 12288 does not fit the LDS
    assert call_with(4, 4096, 4096, 2, 5, 0)[0] == ERR_ARG     # 5 waves: not a variant
    assert call_with(4, 4096, 4096, 3, 1, 0)[0] == ERR_ARG     # no such kernel
    status, message = call_with(1, 4096, 4096, 2, 8, 0)         # M = 1 takes the decode kernel
    assert status == ERR_ARG and "2 <= M <= 8" in message
    status, message = call_with(4, 4096, 4096, 0, 1, 2)         # x-first flag must be 0 or 1
    assert status == ERR_ARG and "does not fit" in message
    assert call_with(4, 4096, 12288, 0, 1, 1)[0] == ERR_PROVIDER  # fits: stops at the device check


def test_gemv_q8_1_refuses_what_it_does_not_run():
    """tensor_gguf_gemv_q8_1_v1 checks encoding and shape before any HIP call (fake device
    addresses; CPU only): a call it runs stops at the device check, which fails with no GPU."""
    manifest = kernels.manifest("gguf_gemv_q8_1", "q4_k", "float32")
    assert [a["name"] for a in manifest["arguments"]] == ["x", "w", "out", "type"]
    assert manifest["arguments"][0]["dtype"] == "float32"
    with pytest.raises(ValueError):
        kernels.manifest("gguf_gemv_q8_1", "q5_k", "float32")

    def call_with(m, n, k, code, x_dtype=11, block=(256, 144)):
        qk, size = block
        shapes = {0: (m, k), 1: (n, k // qk * size), 2: (m, n)}
        dtypes, sizes = {0: x_dtype, 1: 3, 2: 11}, {0: 4 if x_dtype == 11 else 2, 1: 1, 2: 4}
        keep, args = [], (abi.Argument * 4)()
        for j in range(3):
            shape = shapes[j]
            arrays = ((c.c_int64 * 2)(*shape), (c.c_int64 * 2)(sizes[j] * shape[1], sizes[j]))
            keep.append(arrays)
            args[j].kind, args[j].dtype = 1, dtypes[j]
            args[j].buffer = abi.BufferDescriptor(0x10000 * (j + 1), int(np.prod(shape)) * sizes[j], arrays[0],
                                                  arrays[1], 2, dtypes[j], 10, 0)
        args[3].kind, args[3].dtype, args[3].scalar = 2, 7, code
        call = abi.CallDescriptor(1, 72, args, 4, 0, (c.c_uint32 * 3)(1, 1, 1), (c.c_uint32 * 3)(256, 1, 1), 0,
                                  abi.StreamDescriptor(10, 0, 0))
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_gemv_q8_1_v1")(c.byref(call), c.byref(error))
        return status, error.message.decode()

    status, message = call_with(1, 64, 4096, 13, block=(256, 176))      # Q5_K: no Q8_1 dot product
    assert status == ERR_ARG and "Q8_1" in message
    assert call_with(9, 64, 4096, 12)[0] == ERR_ARG                      # M > 8
    assert call_with(8, 64, 16384, 12)[0] == ERR_ARG                     # M * K beyond the LDS
    assert call_with(1, 64, 4096, 12)[0] == ERR_PROVIDER                 # runs: stops at the device
    assert call_with(8, 64, 12288, 14, x_dtype=10, block=(256, 210))[0] == ERR_PROVIDER
    assert call_with(2, 64, 1024, 2, block=(32, 18))[0] == ERR_PROVIDER  # Q4_0


def test_gemm_forced_plan_refuses_a_plan_that_does_not_fit():
    """tensor_gguf_gemm_group_plan_v1 checks the named tile and split against the shape before any
    HIP call (fake device addresses; CPU only)."""
    from tensor_amd.gguf import kernels as gguf_kernels

    manifest = gguf_kernels.manifest("gguf_gemm_group_plan", "q4_k", "float16", count=1)
    names = [a["name"] for a in manifest["arguments"]]
    assert names == ["x", "w0", "out0", "workspace", "type", "tile", "splits"]
    m, n, k = 256, 4096, 4096
    shapes = {"x": (m, k), "w0": (n, k // 256 * 144), "out0": (m, n), "workspace": (1 << 20,)}
    dtypes = {"x": 10, "w0": 3, "out0": 10, "workspace": 3}
    sizes = {"x": 2, "w0": 1, "out0": 2, "workspace": 1}

    def call_with(tile, splits):
        keep, args = [], (abi.Argument * 7)()
        for j, name in enumerate(names[:4]):
            shape = shapes[name]
            strides = [sizes[name]] * len(shape)
            for axis in range(len(shape) - 2, -1, -1):
                strides[axis] = strides[axis + 1] * shape[axis + 1]
            arrays = ((c.c_int64 * len(shape))(*shape), (c.c_int64 * len(shape))(*strides))
            keep.append(arrays)
            args[j].kind, args[j].dtype = 1, dtypes[name]
            args[j].buffer = abi.BufferDescriptor(0x10000 * (j + 1), int(np.prod(shape)) * sizes[name], arrays[0],
                                                  arrays[1], len(shape), dtypes[name], 10, 0)
        for j, value in ((4, 12), (5, tile), (6, splits)):
            args[j].kind, args[j].dtype, args[j].scalar = 2, 7, value
        call = abi.CallDescriptor(1, 72, args, 7, 0, (c.c_uint32 * 3)(1, 1, 1), (c.c_uint32 * 3)(256, 1, 1), 0,
                                  abi.StreamDescriptor(10, 0, 0))
        error = abi.ErrorDescriptor()
        status = _native.kernel("tensor_gguf_gemm_group_plan_v1")(c.byref(call), c.byref(error))
        return status, error.message.decode()

    assert call_with(99, 1)[0] == ERR_ARG          # no such tile
    assert call_with(0, 3)[0] == ERR_ARG           # 64 K steps do not split 3 ways
    status, message = call_with(0, 8)              # 8 x 256 x 4096 x 4 B of partials > 1 MiB
    assert status == ERR_ARG and "workspace" in message
