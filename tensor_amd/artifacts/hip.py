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


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ArtifactError(message)


def _is_name(value) -> bool:
    return isinstance(value, str) and NAME.fullmatch(value) is not None


def _extent(value, symbols: dict, what: str, *, low: int = 1, high: int | None = None) -> None:
    """An extent is an integer in [low, high) or an integer expression over the symbols; an
    expression is evaluated once with every symbol at 1024 (no Python eval), so a reference
    to an undeclared symbol or a malformed node is refused here."""
    try:
        evaluate(value, dict.fromkeys(symbols, 1024))
    except (ValueError, TypeError, KeyError, ZeroDivisionError) as exc:
        raise ArtifactError(f"{what}: invalid expression {value!r}: {exc}") from exc
    if type(value) is int:
        _require(value >= low and (high is None or value < high),
                 f"{what}: {value} is outside [{low}, {high if high is not None else 'inf'})")


# Sections of a manifest, each checked by its own function; a later section may use what an
# earlier one returned (symbols, then the argument table).

def _identity(manifest: dict) -> None:
    _require(manifest.get("format") == FORMAT and manifest.get("format_version") == FORMAT_VERSION,
             f"unsupported format/version: expected {FORMAT} {FORMAT_VERSION}")
    _require(manifest.get("provider") == PROVIDER, f"runtime provider must be {PROVIDER!r}")
    _require(manifest.get("kind") == KIND, f"executable kind must be {KIND!r} for this provider")
    target = manifest.get("target")
    _require(isinstance(target, str) and TARGET.fullmatch(target) is not None, f"invalid gfx target {target!r}")
    try:
        check_requirement(manifest.get("runtime_abi"))
    except ValueError as exc:
        raise ArtifactError(str(exc)) from exc
    compiler = manifest.get("compiler")
    _require(isinstance(compiler, dict) and all(isinstance(compiler.get(k), str) for k in ("name", "version")),
             "compiler provenance needs a name and a version")
    _require(_is_name(manifest.get("entrypoint")), "the entrypoint must be an identifier")


def _symbols(manifest: dict) -> dict:
    symbols = manifest.get("symbols", {})
    _require(isinstance(symbols, dict) and len(symbols) <= 128, "symbols must be a table of at most 128")
    for name, dtype in symbols.items():
        _require(_is_name(name) and dtype in INTEGER_TYPES, f"invalid dimension symbol {name!r}: {dtype!r}")
    return symbols


def _launch(manifest: dict, symbols: dict) -> None:
    launch = manifest.get("launch")
    _require(isinstance(launch, dict) and set(launch) == {"grid", "block", "shared_memory_bytes"},
             "launch needs exactly grid, block and shared_memory_bytes")
    for field in ("grid", "block"):
        dims = launch[field]
        _require(isinstance(dims, list) and len(dims) == 3, f"launch {field} needs three dimensions")
        for dim in dims:
            _extent(dim, symbols, f"launch {field} (positive int32)", high=1 << 31)
    block = launch["block"]
    if all(type(v) is int for v in block):
        _require(block[0] * block[1] * block[2] <= 1024, "a launch block holds at most 1024 threads")
    _extent(launch["shared_memory_bytes"], symbols, "shared memory bytes", low=0, high=160 * 1024 + 1)


def _argument_table(manifest: dict, symbols: dict) -> dict:
    """name -> descriptor of every frontend argument, buffers checked for dtype, shape and a
    power-of-two alignment, scalars for a dtype matching their symbol."""
    arguments = manifest.get("arguments")
    _require(isinstance(arguments, list) and 0 < len(arguments) <= 256, "arguments: 1 to 256 descriptors")
    table = {}
    for argument in arguments:
        _require(isinstance(argument, dict), "an argument descriptor must be an object")
        kind = argument.get("kind", "buffer")
        expected = {"kind", "name", "dtype"} | ({"shape", "alignment"} if kind == "buffer" else set())
        _require(kind in ("buffer", "scalar") and set(argument) == expected,
                 f"argument descriptor fields must be {sorted(expected)}")
        name, dtype = argument["name"], argument["dtype"]
        _require(_is_name(name), f"argument name {name!r} is not an identifier")
        _require(name not in table, f"duplicate argument {name}")
        if kind == "scalar":
            _require(dtype in SCALAR_TYPES and symbols.get(name, dtype) == dtype, f"scalar {name}: bad dtype {dtype!r}")
        else:
            _require(dtype in BUFFER_DTYPES, f"buffer {name}: unsupported dtype {dtype!r}")
            _require(name not in symbols, f"buffer {name} shadows a dimension symbol")
            shape = argument["shape"]
            _require(isinstance(shape, list) and 0 < len(shape) <= 64, f"buffer {name}: shape of rank 1 to 64")
            for dim in shape:
                _extent(dim, symbols, f"buffer {name} shape")
            alignment = argument["alignment"]
            _require(type(alignment) is int and 0 < alignment <= 4096 and not alignment & (alignment - 1),
                     f"buffer {name}: alignment must be a power of two up to 4096")
        table[name] = argument
    _require(any(a.get("kind", "buffer") == "buffer" for a in table.values()), "no buffer arguments")
    return table


def _outputs(manifest: dict, table: dict) -> None:
    outputs = manifest.get("outputs", [])
    buffers = {n for n, a in table.items() if a.get("kind", "buffer") == "buffer"}
    _require(isinstance(outputs, list) and len(outputs) == len(set(outputs)) and set(outputs) <= buffers,
             "each output must name a distinct buffer argument")


def _kernel_abi(manifest: dict, table: dict, symbols: dict) -> None:
    """The kernel's own argument list: every frontend buffer once, scalars either frontend
    arguments or dimension symbols, each with the frontend's kind and dtype."""
    abi = manifest.get("abi")
    _require(isinstance(abi, list) and 0 < len(abi) <= 256, "kernel ABI: 1 to 256 entries")
    seen = set()
    for item in abi:
        _require(isinstance(item, dict) and set(item) == {"kind", "name", "dtype"},
                 "a kernel ABI entry has exactly kind, name and dtype")
        name = item["name"]
        frontend = table.get(name)
        if frontend is not None:
            _require((item["kind"], item["dtype"]) == (frontend.get("kind", "buffer"), frontend["dtype"]),
                     f"kernel ABI entry {name} does not match frontend argument")
        else:
            _require(item["kind"] == "scalar" and symbols.get(name) == item["dtype"],
                     f"unmapped kernel ABI argument {name}")
        _require(name not in seen, f"duplicate kernel ABI entry {name}")
        seen.add(name)
    missing = sorted(n for n, a in table.items() if a.get("kind", "buffer") == "buffer" and n not in seen)
    _require(not missing, f"missing kernel buffer ABI argument(s) {missing}")


def _provenance_and_payloads(manifest: dict) -> None:
    digest = manifest.get("source_sha256")
    _require(isinstance(digest, str) and HASH.fullmatch(digest) is not None, "source_sha256 must be 64 hex digits")
    _require(isinstance(manifest.get("op_set", []), list), "op_set must be a list")
    files = manifest.get("files")
    _require(isinstance(files, dict) and IMAGE in files, f"files must list the payload {IMAGE}")
    for name, value in files.items():
        _require(isinstance(name, str) and (name == IMAGE or re.fullmatch(r"licenses/[A-Za-z0-9_.-]+", name)),
                 f"invalid payload name {name!r}")
        _require(isinstance(value, str) and HASH.fullmatch(value) is not None, f"invalid payload hash for {name}")


def validate_manifest(manifest: object) -> dict:
    """Schema of a `hip` bundle manifest: the reference's manifest fields (format.py:35-266)
    restricted to this provider, checked section by section."""
    _require(isinstance(manifest, dict), "manifest must be an object")
    _identity(manifest)
    symbols = _symbols(manifest)
    _launch(manifest, symbols)
    table = _argument_table(manifest, symbols)
    _outputs(manifest, table)
    _kernel_abi(manifest, table, symbols)
    _provenance_and_payloads(manifest)
    return manifest


# ---------------------------------------------------------- code objects --

def code_object_metadata(image: bytes) -> dict:
    """The AMDGPU metadata note of a 64-bit ELF code object, decoded (its ``amdhsa.target``
    and one record per kernel in ``amdhsa.kernels``: arguments, LDS, scratch, registers)."""
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
                    if not isinstance(metadata, dict):
                        raise ValueError("metadata is not a map")
                    return metadata
    except (struct.error, KeyError, TypeError, ValueError) as exc:
        raise ArtifactError(f"unreadable code object metadata: {exc}") from exc
    raise ArtifactError(f"{IMAGE} carries no AMDGPU kernel metadata")


def code_object_kernels(image: bytes) -> tuple[str, dict]:
    """(target, {kernel name: [explicit arguments]}) from a gfx950 ELF code object's
    AMDGPU metadata note; each argument is (value_kind, size)."""
    metadata = code_object_metadata(image)
    try:
        kernels = {}
        for kernel in metadata.get("amdhsa.kernels", []):
            kernels[kernel[".name"]] = [(a.get(".value_kind"), a.get(".size")) for a in kernel.get(".args", [])
                                        if not str(a.get(".value_kind", "")).startswith("hidden_")]
    except (KeyError, TypeError, AttributeError) as exc:
        raise ArtifactError(f"unreadable code object metadata: {exc}") from exc
    return metadata.get("amdhsa.target", ""), kernels


def offload_code_objects(image: bytes, target: str = "gfx950") -> list:
    """The device code objects for ``target`` inside a host shared library built by hipcc:
    its ``.hip_fatbin`` section holds one clang offload bundle per translation unit (a
    24-byte magic, an entry count, then offset, size and triple of each entry)."""
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    if image[:4] != b"\x7fELF" or len(image) < 64:
        raise ArtifactError("not an ELF shared library")
    shoff, = struct.unpack_from("<Q", image, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", image, 0x3A)
    sections = [struct.unpack_from("<IIQQQQ", image, shoff + i * shentsize) for i in range(shnum)]
    names = sections[shstrndx][4]
    fatbin = None
    for name_offset, _, _, _, offset, size in sections:
        name = image[names + name_offset:image.index(b"\0", names + name_offset)]
        if name == b".hip_fatbin":
            fatbin = image[offset:offset + size]
    if fatbin is None:
        raise ArtifactError("no .hip_fatbin section")
    objects, position = [], 0
    while (start := fatbin.find(magic, position)) >= 0:
        count, = struct.unpack_from("<Q", fatbin, start + len(magic))
        entry = start + len(magic) + 8
        for _ in range(count):
            offset, size, triple_size = struct.unpack_from("<QQQ", fatbin, entry)
            triple = fatbin[entry + 24:entry + 24 + triple_size].decode()
            entry += 24 + triple_size
            if triple.endswith("--" + target) and size:
                objects.append(fatbin[start + offset:start + offset + size])
        position = start + len(magic)
    return objects


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
