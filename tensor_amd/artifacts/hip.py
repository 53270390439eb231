"""`hip` executable bundles: hand-built gfx950 code objects the provider loads.

The container is the reference's executable bundle (src/tensor/artifacts/format.py:1-357):
a zip archive holding ``manifest.json`` and the payload files it lists with their
SHA-256, every member verified before any byte reaches the HIP runtime.  The
manifest keeps the reference's launch, argument, output and kernel-ABI schema
(``format: "tensor.module"``, version 3) with ``provider: "hip"`` and
``kind: "hsaco"``; the payload is ``kernel.hsaco``, an unbundled gfx950 ELF code
object (``hipcc --genco --no-gpu-bundle-output``).  The TileLang provenance fields
and ``kernel.tirx.json`` the reference requires of compiler-produced bundles
(format.py:253-263, :287-288) do not apply to hand-written kernels; in their
place the loader checks the manifest's kernel ABI against the argument metadata
the code object itself carries (its AMDGPU note), so a manifest that does not
match its kernel is rejected before launch instead of passing wrong parameters.
"""

from __future__ import annotations

import hashlib
import io
import json
import re
import struct
import zipfile
from pathlib import Path

from tensor_amd.runtime.abi import check_requirement
from tensor_amd.runtime.signature import INTEGER_TYPES, SCALAR_TYPES, evaluate

FORMAT = "tensor.module"
FORMAT_VERSION = 3
PROVIDER, KIND, IMAGE = "hip", "hsaco", "kernel.hsaco"
MAX_UNCOMPRESSED = 128 * 1024 * 1024
MAX_MANIFEST = 2 * 1024 * 1024
NAME = re.compile(r"[A-Za-z_]\w*\Z")
HASH = re.compile(r"[0-9a-f]{64}\Z")
TARGET = re.compile(r"gfx[0-9a-f]{3,4}\Z")
BUFFER_DTYPES = {*SCALAR_TYPES, "float16", "bfloat16"}
SCALAR_BYTES = {"bool": 1, "int8": 1, "uint8": 1, "int16": 2, "uint16": 2, "int32": 4, "uint32": 4,
                "int64": 8, "uint64": 8, "float32": 4, "float64": 8}


class ArtifactError(ValueError):
    pass


def _expression(value, symbols: dict) -> None:
    """Integers, symbol references and bounded integer expressions (no Python eval)."""
    probe = {name: 1024 for name in symbols}
    try:
        evaluate(value, probe)
    except (ValueError, TypeError, KeyError, ZeroDivisionError) as exc:
        raise ArtifactError(f"invalid expression {value!r}: {exc}") from exc


def validate_manifest(manifest: object) -> dict:
    """Schema of a `hip` bundle manifest (format.py:35-266, restricted to this provider)."""
    if not isinstance(manifest, dict):
        raise ArtifactError("manifest must be an object")
    if manifest.get("format") != FORMAT or manifest.get("format_version") != FORMAT_VERSION:
        raise ArtifactError("unsupported Tensor artifact format/version")
    if manifest.get("provider") != PROVIDER:
        raise ArtifactError("unsupported runtime provider")
    if manifest.get("kind") != KIND:
        raise ArtifactError("invalid executable kind for provider")
    if not isinstance(manifest.get("target"), str) or not TARGET.fullmatch(manifest["target"]):
        raise ArtifactError("invalid provider target")
    try:
        check_requirement(manifest.get("runtime_abi"))
    except ValueError as exc:
        raise ArtifactError(str(exc)) from exc
    compiler = manifest.get("compiler")
    if not isinstance(compiler, dict) or not isinstance(compiler.get("name"), str) or not isinstance(
            compiler.get("version"), str):
        raise ArtifactError("missing compiler provenance")
    entrypoint = manifest.get("entrypoint")
    if not isinstance(entrypoint, str) or not NAME.fullmatch(entrypoint):
        raise ArtifactError("invalid executable entrypoint")
    symbols = manifest.get("symbols", {})
    if not isinstance(symbols, dict) or len(symbols) > 128 or any(
            not isinstance(n, str) or not NAME.fullmatch(n) or d not in INTEGER_TYPES for n, d in symbols.items()):
        raise ArtifactError("invalid dimension symbols")
    launch = manifest.get("launch")
    if not isinstance(launch, dict) or set(launch) != {"grid", "block", "shared_memory_bytes"}:
        raise ArtifactError("invalid launch description")
    for field in ("grid", "block"):
        dims = launch[field]
        if not isinstance(dims, list) or len(dims) != 3:
            raise ArtifactError(f"{field} must contain three dimensions")
        for extent in dims:
            _expression(extent, symbols)
            if type(extent) is int and not 1 <= extent < (1 << 31):
                raise ArtifactError(f"{field} must have positive int32 dimensions")
    if all(type(v) is int for v in launch["block"]) and launch["block"][0] * launch["block"][1] * launch["block"][2] > 1024:
        raise ArtifactError("launch block exceeds 1024 threads")
    _expression(launch["shared_memory_bytes"], symbols)
    shared = launch["shared_memory_bytes"]
    if type(shared) is int and not 0 <= shared <= 160 * 1024:
        raise ArtifactError("invalid shared memory size")
    arguments = manifest.get("arguments")
    if not isinstance(arguments, list) or not arguments or len(arguments) > 256:
        raise ArtifactError("invalid artifact argument count")
    names, buffers = [], set()
    for argument in arguments:
        if not isinstance(argument, dict):
            raise ArtifactError("invalid argument")
        kind = argument.get("kind", "buffer")
        fields = {"kind", "name", "dtype", "shape", "alignment"} if kind == "buffer" else {"kind", "name", "dtype"}
        if set(argument) != fields or kind not in ("buffer", "scalar"):
            raise ArtifactError("invalid argument descriptor")
        name, dtype = argument["name"], argument["dtype"]
        if not isinstance(name, str) or not NAME.fullmatch(name):
            raise ArtifactError("invalid argument name")
        if kind == "scalar":
            if dtype not in SCALAR_TYPES or (name in symbols and symbols[name] != dtype):
                raise ArtifactError("invalid scalar argument dtype")
        else:
            if dtype not in BUFFER_DTYPES:
                raise ArtifactError(f"unsupported argument dtype {dtype}")
            if name in symbols:
                raise ArtifactError("buffer and dimension names must be distinct")
            buffers.add(name)
            shape = argument["shape"]
            if not isinstance(shape, list) or not shape or len(shape) > 64:
                raise ArtifactError("invalid buffer shape")
            for extent in shape:
                _expression(extent, symbols)
                if type(extent) is int and extent < 1:
                    raise ArtifactError("invalid buffer shape")
            alignment = argument["alignment"]
            if type(alignment) is not int or not 1 <= alignment <= 4096 or alignment & (alignment - 1):
                raise ArtifactError("invalid buffer alignment")
        names.append(name)
    if len(names) != len(set(names)):
        raise ArtifactError("duplicate argument")
    if not buffers:
        raise ArtifactError("artifact has no buffer arguments")
    outputs = manifest.get("outputs", [])
    if not isinstance(outputs, list) or any(n not in buffers for n in outputs) or len(outputs) != len(set(outputs)):
        raise ArtifactError("invalid output names")
    abi = manifest.get("abi")
    if not isinstance(abi, list) or not abi or len(abi) > 256:
        raise ArtifactError("missing or invalid kernel ABI")
    frontend = {item["name"]: item for item in arguments}
    abi_names = []
    for item in abi:
        if not isinstance(item, dict) or set(item) != {"kind", "name", "dtype"}:
            raise ArtifactError("invalid kernel ABI argument")
        name, kind, dtype = item["name"], item["kind"], item["dtype"]
        original = frontend.get(name)
        if original is not None:
            if kind != original.get("kind", "buffer") or dtype != original["dtype"]:
                raise ArtifactError("kernel ABI does not match frontend argument")
        elif kind != "scalar" or symbols.get(name) != dtype:
            raise ArtifactError(f"unmapped kernel ABI argument {name}")
        abi_names.append(name)
    if len(abi_names) != len(set(abi_names)) or buffers - set(abi_names):
        raise ArtifactError("duplicate or missing kernel buffer ABI argument")
    value = manifest.get("source_sha256")
    if not isinstance(value, str) or not HASH.fullmatch(value):
        raise ArtifactError("invalid source_sha256")
    if not isinstance(manifest.get("op_set", []), list):
        raise ArtifactError("invalid frontend operator set")
    files = manifest.get("files")
    if not isinstance(files, dict) or IMAGE not in files:
        raise ArtifactError("missing executable payload")
    for name, digest in files.items():
        if not isinstance(name, str) or not (name == IMAGE or re.fullmatch(r"licenses/[A-Za-z0-9_.-]+", name)):
            raise ArtifactError(f"invalid payload name: {name}")
        if not isinstance(digest, str) or not HASH.fullmatch(digest):
            raise ArtifactError(f"invalid payload hash: {name}")
    return manifest


# ---------------------------------------------------------- code objects --

def code_object_kernels(image: bytes) -> tuple[str, dict]:
    """(target, {kernel name: [explicit arguments]}) from a gfx950 ELF code object's
    AMDGPU metadata note; each argument is (value_kind, size)."""
    import msgpack

    if image[:4] != b"\x7fELF" or len(image) < 64 or image[4] != 2 or image[5] != 1:
        raise ArtifactError(f"{IMAGE} is not a 64-bit little-endian ELF code object")
    try:
        shoff, = struct.unpack_from("<Q", image, 0x28)
        shentsize, shnum = struct.unpack_from("<HH", image, 0x3A)
        for index in range(shnum):
            _, sh_type, _, _, offset, size = struct.unpack_from("<IIQQQQ", image, shoff + index * shentsize)
            if sh_type != 7:  # SHT_NOTE
                continue
            position, end = offset, offset + size
            while position + 12 <= end:
                namesz, descsz, note_type = struct.unpack_from("<III", image, position)
                position += 12
                name = image[position:position + namesz]
                position += (namesz + 3) & ~3
                desc = image[position:position + descsz]
                position += (descsz + 3) & ~3
                if name.rstrip(b"\0") == b"AMDGPU" and note_type == 32:  # NT_AMDGPU_METADATA
                    metadata = msgpack.unpackb(desc, raw=False)
                    target = metadata.get("amdhsa.target", "")
                    kernels = {}
                    for kernel in metadata.get("amdhsa.kernels", []):
                        kernels[kernel[".name"]] = [(a.get(".value_kind"), a.get(".size")) for a in kernel.get(".args", [])
                                                    if not str(a.get(".value_kind", "")).startswith("hidden_")]
                    return target, kernels
    except (struct.error, KeyError, TypeError, ValueError) as exc:
        raise ArtifactError(f"unreadable code object metadata: {exc}") from exc
    raise ArtifactError(f"{IMAGE} carries no AMDGPU kernel metadata")


def check_kernel(manifest: dict, image: bytes) -> None:
    """The code object must target the manifest's target and hold the entry point with
    exactly the manifest's kernel ABI: a buffer is a global pointer, a scalar a value of its
    dtype's size."""
    target, kernels = code_object_kernels(image)
    if not target.endswith("--" + manifest["target"]) and not target.endswith("-" + manifest["target"]):
        raise ArtifactError(f"code object target {target} does not match {manifest['target']}")
    entry = manifest["entrypoint"]
    if entry not in kernels:
        raise ArtifactError(f"code object has no kernel {entry}")
    explicit = kernels[entry]
    abi = manifest["abi"]
    if len(explicit) != len(abi):
        raise ArtifactError(f"kernel {entry} takes {len(explicit)} arguments, the manifest ABI lists {len(abi)}")
    for position, ((value_kind, size), item) in enumerate(zip(explicit, abi)):
        if item["kind"] == "buffer":
            ok = value_kind == "global_buffer" and size == 8
        else:
            ok = value_kind == "by_value" and size == SCALAR_BYTES[item["dtype"]]
        if not ok:
            raise ArtifactError(f"kernel {entry} argument {position} ({value_kind}, {size} B) does not match "
                                f"the manifest's {item['kind']} {item['name']}: {item['dtype']}")


# ---------------------------------------------------------------- bundles --

def read_artifact(path: str | Path) -> tuple[dict, dict[str, bytes]]:
    """Verify every member (names, sizes, hashes, manifest schema, kernel ABI) before
    any binary is handed to the HIP runtime (format.py:268-357)."""
    try:
        with zipfile.ZipFile(path) as archive:
            members = archive.infolist()
            names = [item.filename for item in members]
            if len(names) != len(set(names)) or len(names) > 1024:
                raise ArtifactError("duplicate or excessive archive members")
            if sum(item.file_size for item in members) > MAX_UNCOMPRESSED:
                raise ArtifactError("artifact exceeds the 128 MiB limit")
            if "manifest.json" not in names or archive.getinfo("manifest.json").file_size > MAX_MANIFEST:
                raise ArtifactError("missing or oversized manifest")
            manifest = validate_manifest(json.loads(archive.read("manifest.json")))
            if set(names) != {"manifest.json", *manifest["files"]}:
                raise ArtifactError("archive members do not match the manifest")
            files = {name: archive.read(name) for name in manifest["files"]}
    except (zipfile.BadZipFile, KeyError, json.JSONDecodeError, UnicodeDecodeError, OSError) as exc:
        raise ArtifactError(f"invalid artifact: {exc}") from exc
    for name, content in files.items():
        if hashlib.sha256(content).hexdigest() != manifest["files"][name]:
            raise ArtifactError(f"payload hash mismatch: {name}")
    check_kernel(manifest, files[IMAGE])
    return manifest, files


def write_artifact(path: str | Path, image: bytes, *, entrypoint: str, arguments: list, launch: dict,
                   abi: list | None = None, symbols: dict | None = None, outputs: list | None = None,
                   target: str = "gfx950", compiler: dict | None = None, source: bytes = b"",
                   op_set: list | None = None, name: str | None = None,
                   capabilities: tuple = ("contiguous", "executable_descriptors", "no_external_workspace",
                                          "scalars")) -> dict:
    """Pack a code object and its manifest into a bundle; returns the manifest.  The bundle is
    validated with the same checks ``read_artifact`` applies before it is written."""
    manifest = {
        "format": FORMAT,
        "format_version": FORMAT_VERSION,
        "provider": PROVIDER,
        "kind": KIND,
        "target": target,
        "runtime_abi": {"major": 1, "minor": 1, "required_capabilities": list(capabilities)},
        "compiler": compiler or {"name": "hipcc", "version": "unknown"},
        "entrypoint": entrypoint,
        "symbols": symbols or {},
        "launch": launch,
        "arguments": arguments,
        "outputs": outputs or [],
        "abi": abi if abi is not None else [{"kind": a.get("kind", "buffer"), "name": a["name"], "dtype": a["dtype"]}
                                            for a in arguments],
        "source_sha256": hashlib.sha256(source).hexdigest(),
        "op_set": op_set or [],
        "files": {IMAGE: hashlib.sha256(image).hexdigest()},
    }
    if name:
        manifest["name"] = name
    validate_manifest(manifest)
    check_kernel(manifest, image)
    buffer = io.BytesIO()
    with zipfile.ZipFile(buffer, "w", zipfile.ZIP_DEFLATED) as archive:
        archive.writestr("manifest.json", json.dumps(manifest, indent=1, sort_keys=True))
        archive.writestr(IMAGE, image)
    Path(path).write_bytes(buffer.getvalue())
    return manifest
