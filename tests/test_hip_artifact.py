"""`hip` executable bundles (tensor_amd.artifacts.hip) on the CPU: schema, tamper checks, the
kernel-ABI check against the code object's own metadata, and the argument checks of the
module launch entry that run before any HIP call.  The bundle format follows the
reference's (src/tensor/artifacts/format.py); the checks mirror its tests of malformed
bundles."""

from __future__ import annotations

import copy
import ctypes as c
import hashlib
import io
import json
import zipfile

import pytest

from tensor_amd import _native
from tensor_amd.artifacts import ArtifactError, read_artifact, validate_manifest, write_artifact
from tensor_amd.artifacts.hip import code_object_kernels
from tensor_amd.kernels import BUNDLES, bundle_path
from tensor_amd.runtime import abi


@pytest.fixture(scope="module")
def swiglu():
    """The built SwiGLU bundle (built here if the package build has not run yet)."""
    path = bundle_path("swiglu")
    if not path.exists():
        from tensor_amd import build

        build.build_bundles()
    manifest, files = read_artifact(path)
    return path, manifest, files


def repack(manifest, files, extra=None):
    buffer = io.BytesIO()
    with zipfile.ZipFile(buffer, "w") as archive:
        archive.writestr("manifest.json", json.dumps(manifest))
        for name, content in files.items():
            archive.writestr(name, content)
        for name, content in (extra or {}).items():
            archive.writestr(name, content)
    return buffer.getvalue()


def test_bundle_round_trip(swiglu, tmp_path):
    path, manifest, files = swiglu
    assert manifest["provider"] == "hip" and manifest["kind"] == "hsaco" and manifest["target"] == "gfx950"
    assert manifest["entrypoint"] == BUNDLES["swiglu"]["entrypoint"]
    assert manifest["files"]["kernel.hsaco"] == hashlib.sha256(files["kernel.hsaco"]).hexdigest()
    target, kernels = code_object_kernels(files["kernel.hsaco"])
    assert target.endswith("gfx950")
    # gate, up, out as global pointers, then M and N by value (4 bytes each)
    assert kernels["tensor_swiglu_f16"] == [("global_buffer", 8)] * 3 + [("by_value", 4)] * 2
    again = tmp_path / "again.tbin"
    spec = BUNDLES["swiglu"]
    write_artifact(again, files["kernel.hsaco"], target="gfx950", compiler=manifest["compiler"], **spec)
    assert read_artifact(again)[0]["abi"] == manifest["abi"]


@pytest.mark.parametrize("change,needle", [
    (lambda m: m.update(provider="cuda"), "provider"),
    (lambda m: m.update(kind="cubin"), "kind"),
    (lambda m: m.update(target="sm_90"), "target"),
    (lambda m: m.update(format_version=9), "format"),
    (lambda m: m.update(entrypoint="not a name"), "entrypoint"),
    (lambda m: m["runtime_abi"].update(major=2), "ABI"),
    (lambda m: m["launch"].update(block=[1024, 2, 1]), "1024"),
    (lambda m: m["launch"].update(grid=[0, 1, 1]), "positive"),
    (lambda m: m["launch"].update(grid=[{"var": "Q"}, 1, 1]), "expression"),
    (lambda m: m["arguments"][0].update(alignment=3), "alignment"),
    (lambda m: m["arguments"][1].update(name="gate"), "duplicate"),
    (lambda m: m.update(outputs=["M"]), "output"),
    (lambda m: m["abi"].pop(0), "missing kernel buffer"),
    (lambda m: m["abi"][0].update(dtype="float32"), "does not match frontend"),
    (lambda m: m["abi"].append({"kind": "scalar", "name": "K", "dtype": "uint32"}), "unmapped"),
    (lambda m: m.update(source_sha256="xyz"), "source_sha256"),
    (lambda m: m["files"].update({"../escape": "0" * 64}), "payload name"),
])
def test_manifest_schema_rejections(swiglu, change, needle):
    _, manifest, _ = swiglu
    bad = copy.deepcopy(manifest)
    change(bad)
    with pytest.raises(ArtifactError, match=needle):
        validate_manifest(bad)


def test_tampered_bundles_are_rejected_before_loading(swiglu, tmp_path):
    _, manifest, files = swiglu
    cases = {}
    image = bytearray(files["kernel.hsaco"])
    image[-1] ^= 0xFF
    cases["hash mismatch"] = repack(manifest, {"kernel.hsaco": bytes(image)})
    cases["do not match"] = repack(manifest, files, extra={"licenses/EXTRA": b"x"})
    wrong = copy.deepcopy(manifest)
    wrong["files"]["kernel.hsaco"] = hashlib.sha256(b"not an elf" * 10).hexdigest()
    cases["not a 64-bit"] = repack(wrong, {"kernel.hsaco": b"not an elf" * 10})
    cases["invalid artifact"] = b"this is not a zip archive"
    for needle, blob in cases.items():
        path = tmp_path / "bad.tbin"
        path.write_bytes(blob)
        with pytest.raises(ArtifactError, match=needle):
            read_artifact(path)


def _n_as_uint64(m):
    m["symbols"]["N"] = "uint64"
    m["abi"][4]["dtype"] = "uint64"


@pytest.mark.parametrize("change,needle", [
    (_n_as_uint64, "argument 4"),  # the kernel takes N as 4 bytes; 8 would shift nothing but misread
    (lambda m: m["abi"].pop(4), "takes 5 arguments"),
    (lambda m: m.update(entrypoint="tensor_swiglu_f32"), "no kernel"),
    (lambda m: m.update(target="gfx942"), "target"),
])
def test_kernel_abi_must_match_the_code_object(swiglu, tmp_path, change, needle):
    """A manifest whose ABI disagrees with the kernel's own argument metadata is refused, so a
    wrongly described kernel never receives parameters it does not expect."""
    _, manifest, files = swiglu
    bad = copy.deepcopy(manifest)
    change(bad)
    validate_manifest(bad)  # the schema alone accepts it
    path = tmp_path / "bad.tbin"
    path.write_bytes(repack(bad, files))
    with pytest.raises(ArtifactError, match=needle):
        read_artifact(path)


class ModuleCall:
    """A well-formed module call (fake, never dereferenced addresses)."""

    def __init__(self):
        self.shape = (c.c_int64 * 1)(64)
        self.strides = (c.c_int64 * 1)(2)
        self.args = (abi.Argument * 2)()
        self.args[0].kind, self.args[0].dtype = 1, 10
        self.args[0].buffer = abi.BufferDescriptor(0x10000, 128, self.shape, self.strides, 1, 10, 10, 0)
        self.args[1].kind, self.args[1].dtype, self.args[1].scalar = 2, 7, 64
        self.call = abi.CallDescriptor(1, 72, self.args, 2, 0, (c.c_uint32 * 3)(1, 1, 1),
                                       (c.c_uint32 * 3)(256, 1, 1), 0, abi.StreamDescriptor(10, 0, 0))

    def run(self, function=0x1234):
        error = abi.ErrorDescriptor()
        status = _native.library().tensor_hip_module_launch_v1(function, c.byref(self.call), c.byref(error))
        return status, error.message.decode()


@pytest.mark.parametrize("mutate,code,needle", [
    (lambda m: setattr(m.call, "abi_version", 2), 1, "ABI"),
    (lambda m: setattr(m.call, "flags", 1), 2, "flags"),
    (lambda m: setattr(m.call, "argument_count", 300), 2, "argument count"),
    (lambda m: setattr(m.call.stream, "device_type", 2), 3, "ROCm stream"),
    (lambda m: m.call.block.__setitem__(0, 2048), 2, "1024"),
    (lambda m: m.call.grid.__setitem__(1, 0), 2, "positive"),
    (lambda m: setattr(m.args[0].buffer, "device_ordinal", 3), 2, "argument 0"),
    (lambda m: setattr(m.args[0].buffer, "device_type", 1), 2, "argument 0"),
    (lambda m: setattr(m.args[1], "kind", 7), 2, "unknown kind"),
])
def test_module_launch_checks_descriptors_before_hip(mutate, code, needle):
    call = ModuleCall()
    mutate(call)
    status, message = call.run()
    assert status == code and needle in message, (status, message)


def test_module_launch_needs_a_function():
    status, message = ModuleCall().run(function=0)
    assert status == 2 and "function" in message
