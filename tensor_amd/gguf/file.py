"""GGUF files: raw block ingestion for the kernels, and a writer.

The reference plans a GGUF reader for raw block ingestion but has none
(research/plans/v1-benchmarks.md:287-313; the showcase takes its bytes from
AKAS's ``sample_weight``, benchmark.py:453-459).  This module follows the public
GGUF specification (ggml's ``docs/gguf.md``; file versions 2 and 3 share one
layout), all little-endian:

    magic "GGUF" | version u32 | tensor_count u64 | metadata_kv_count u64
    metadata: key string | value_type u32 | value            (kv_count times)
    tensor infos: name string | n_dims u32 | ne u64[n_dims] | ggml_type u32 | offset u64
    padding to ``general.alignment`` (u32, default 32)
    tensor data; each tensor at data_start + offset, offset a multiple of the alignment

where a string is a u64 byte length followed by UTF-8 bytes, and ``ne[0]`` is the
innermost extent (a weight's K), so the numpy shape is ``ne`` reversed.  Every
length, count and extent is checked against the file before it is used: a file
is untrusted input.  Tensor data is never copied on read; ``raw`` returns a
read-only view of the memory-mapped file, shaped ``[rows, row_bytes]`` for block
types, which ``Device.from_numpy`` uploads as the kernels' ``w`` argument.
"""

from __future__ import annotations

import math
import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

MAGIC = b"GGUF"
VERSIONS = (2, 3)
DEFAULT_ALIGNMENT = 32
MAX_DIMS = 4  # GGML_MAX_DIMS

# Metadata value types.
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALARS = {
    UINT8: "<u1", INT8: "<i1", UINT16: "<u2", INT16: "<i2", UINT32: "<u4", INT32: "<i4",
    FLOAT32: "<f4", BOOL: "<u1", UINT64: "<u8", INT64: "<i8", FLOAT64: "<f8",
}

# GGML tensor types: code -> (name, elements per block, bytes per block).  Block types are
# the public GGML layouts; the kernels run the four in tensor_amd.gguf.quant.GEOMETRY.
TENSOR_TYPES = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20),
    6: ("q5_0", 32, 22), 7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 9: ("q8_1", 32, 36),
    10: ("q2_k", 256, 84), 11: ("q3_k", 256, 110), 12: ("q4_k", 256, 144), 13: ("q5_k", 256, 176),
    14: ("q6_k", 256, 210), 15: ("q8_k", 256, 292), 24: ("i8", 1, 1), 25: ("i16", 1, 2),
    26: ("i32", 1, 4), 27: ("i64", 1, 8), 28: ("f64", 1, 8), 30: ("bf16", 1, 2),
}
_ELEMENT_DTYPES = {0: "<f4", 1: "<f2", 24: "<i1", 25: "<i2", 26: "<i4", 27: "<i8", 28: "<f8", 30: "<u2"}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file."""


@dataclass(frozen=True)
class Value:
    """A metadata value with an explicit GGUF type (for the writer); ``element_type``
    gives an ARRAY's element type."""

    type: int
    value: object
    element_type: int | None = None


@dataclass(frozen=True)
class TensorInfo:
    name: str
    ne: tuple             # GGML extents, innermost first
    ggml_type: int
    offset: int           # from the start of the data section
    nbytes: int | None    # None for a tensor type this module does not know

    @property
    def shape(self) -> tuple:
        """numpy order (outermost first)."""
        return tuple(reversed(self.ne))

    @property
    def type_name(self) -> str:
        return TENSOR_TYPES.get(self.ggml_type, (f"type{self.ggml_type}",))[0]


def tensor_nbytes(ggml_type: int, ne) -> int:
    name, block, size = TENSOR_TYPES[ggml_type]
    if ne[0] % block:
        raise GGUFError(f"{name} rows need a multiple of {block} elements, not {ne[0]}")
    return ne[0] // block * size * math.prod(ne[1:])


class _Cursor:
    def __init__(self, data, position: int = 0):
        self.data, self.position = data, position

    def take(self, count: int) -> memoryview:
        if count < 0 or self.position + count > len(self.data):
            raise GGUFError(f"truncated file: {count} bytes needed at offset {self.position}")
        view = memoryview(self.data)[self.position:self.position + count]
        self.position += count
        return view

    def unpack(self, fmt: str):
        size = struct.calcsize(fmt)
        return struct.unpack(fmt, self.take(size))[0]

    def string(self) -> str:
        length = self.unpack("<Q")
        try:
            return bytes(self.take(length)).decode("utf-8")
        except UnicodeDecodeError as exc:
            raise GGUFError(f"string at offset {self.position - length} is not UTF-8") from exc

    def value(self, kind: int, depth: int = 0):
        if kind in _SCALARS:
            value = np.frombuffer(self.take(np.dtype(_SCALARS[kind]).itemsize), _SCALARS[kind])[0]
            if kind == BOOL:
                if value > 1:
                    raise GGUFError("bool metadata value is neither 0 nor 1")
                return bool(value)
            return value.item()
        if kind == STRING:
            return self.string()
        if kind == ARRAY:
            if depth:
                raise GGUFError("nested metadata arrays are not supported")
            element, count = self.unpack("<I"), self.unpack("<Q")
            if element in _SCALARS and element != BOOL:
                dtype = np.dtype(_SCALARS[element])
                if count > len(self.data):
                    raise GGUFError("metadata array longer than the file")
                return np.frombuffer(self.take(count * dtype.itemsize), dtype).copy()
            if count > len(self.data) - self.position:  # every element takes at least one byte
                raise GGUFError("metadata array longer than the file")
            return [self.value(element, depth + 1) for _ in range(count)]
        raise GGUFError(f"unknown metadata value type {kind}")


class GGUFFile:
    """A parsed GGUF file over a read-only memory map of it."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as handle:
            size = os.fstat(handle.fileno()).st_size
            if size < 24:
                raise GGUFError("file too small for a GGUF header")
            self._map = mmap.mmap(handle.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse(size)
        except BaseException:
            self.close()
            raise

    def _parse(self, size: int) -> None:
        cursor = _Cursor(self._map)
        if bytes(cursor.take(4)) != MAGIC:
            raise GGUFError("not a GGUF file (bad magic)")
        self.version = cursor.unpack("<I")
        if self.version not in VERSIONS:
            raise GGUFError(f"GGUF version {self.version} is not supported (versions {VERSIONS})")
        tensor_count, kv_count = cursor.unpack("<Q"), cursor.unpack("<Q")
        if tensor_count > size or kv_count > size:
            raise GGUFError("tensor or metadata count larger than the file")
        self.metadata: dict = {}
        self.metadata_types: dict = {}
        for _ in range(kv_count):
            key = cursor.string()
            if key in self.metadata:
                raise GGUFError(f"duplicate metadata key {key!r}")
            kind = cursor.unpack("<I")
            self.metadata[key] = cursor.value(kind)
            self.metadata_types[key] = kind
        alignment = self.metadata.get("general.alignment", DEFAULT_ALIGNMENT)
        if self.metadata_types.get("general.alignment", UINT32) != UINT32 or not isinstance(alignment, int) \
                or alignment < 1 or alignment & (alignment - 1):
            raise GGUFError("general.alignment must be a power-of-two uint32")
        self.alignment = alignment
        infos = []
        for _ in range(tensor_count):
            name = cursor.string()
            n_dims = cursor.unpack("<I")
            if not 1 <= n_dims <= MAX_DIMS:
                raise GGUFError(f"tensor {name!r} has {n_dims} dimensions (1 to {MAX_DIMS} allowed)")
            ne = tuple(cursor.unpack("<Q") for _ in range(n_dims))
            if any(extent < 1 or extent > size * 8 for extent in ne):
                raise GGUFError(f"tensor {name!r} has an impossible extent {ne}")
            ggml_type, offset = cursor.unpack("<I"), cursor.unpack("<Q")
            nbytes = tensor_nbytes(ggml_type, ne) if ggml_type in TENSOR_TYPES else None
            infos.append(TensorInfo(name, ne, ggml_type, offset, nbytes))
        self.data_offset = -(-cursor.position // alignment) * alignment
        self.tensors: dict = {}
        for info in infos:
            if info.name in self.tensors:
                raise GGUFError(f"duplicate tensor name {info.name!r}")
            if info.offset % alignment:
                raise GGUFError(f"tensor {info.name!r} offset {info.offset} is not {alignment}-byte aligned")
            if info.nbytes is not None and self.data_offset + info.offset + info.nbytes > size:
                raise GGUFError(f"tensor {info.name!r} extends past the end of the file")
            self.tensors[info.name] = info

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only view: ``[rows, row_bytes]`` uint8 for block
        types, the element dtype in numpy shape for the others (bf16 as uint16)."""
        info = self.tensors[name]
        if info.nbytes is None:
            raise GGUFError(f"tensor {name!r} has GGML type {info.ggml_type}, which this reader does not know")
        start = self.data_offset + info.offset
        data = np.frombuffer(self._map, np.uint8, info.nbytes, start)
        if info.ggml_type in _ELEMENT_DTYPES:
            return data.view(_ELEMENT_DTYPES[info.ggml_type]).reshape(info.shape)
        rows = math.prod(info.ne[1:])
        return data.reshape(rows, info.nbytes // rows)

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:  # a raw() view is still alive; the map closes with it
                pass
            self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def read(path) -> GGUFFile:
    return GGUFFile(path)


# ------------------------------------------------------------------- writer --

def _infer(value) -> Value:
    if isinstance(value, Value):
        return value
    if isinstance(value, bool):
        return Value(BOOL, value)
    if isinstance(value, int):
        return Value(UINT32 if 0 <= value < 1 << 32 else INT64, value)
    if isinstance(value, float):
        return Value(FLOAT32, value)
    if isinstance(value, str):
        return Value(STRING, value)
    if isinstance(value, np.ndarray):
        kinds = {np.dtype(v): k for k, v in _SCALARS.items() if k != BOOL}
        if value.dtype.newbyteorder("<") not in kinds or value.ndim != 1:
            raise GGUFError(f"no GGUF array type for {value.dtype} arrays of rank {value.ndim}")
        return Value(ARRAY, value, kinds[value.dtype.newbyteorder("<")])
    if isinstance(value, (list, tuple)):
        if not value:
            raise GGUFError("an empty list needs an explicit Value(ARRAY, [], element_type)")
        return Value(ARRAY, list(value), _infer(value[0]).type)
    raise GGUFError(f"no GGUF metadata type for {type(value).__name__}")


def _encode(kind: int, value, element_type=None) -> bytes:
    if kind in _SCALARS:
        return np.array(value, _SCALARS[kind]).tobytes()
    if kind == STRING:
        data = value.encode("utf-8")
        return struct.pack("<Q", len(data)) + data
    if kind == ARRAY:
        if element_type is None or element_type == ARRAY:
            raise GGUFError("arrays need a scalar or string element type")
        head = struct.pack("<IQ", element_type, len(value))
        if element_type in _SCALARS and isinstance(value, np.ndarray):
            return head + np.ascontiguousarray(value, _SCALARS[element_type]).tobytes()
        return head + b"".join(_encode(element_type, item) for item in value)
    raise GGUFError(f"unknown metadata value type {kind}")


def write(path, tensors: dict, metadata: dict | None = None, *, alignment: int = DEFAULT_ALIGNMENT,
          version: int = 3) -> Path:
    """Write a GGUF file.  ``tensors`` maps a name to ``(ggml_type, ne, data)`` with ``ne``
    innermost first and ``data`` the tensor's bytes (any array, written as raw bytes), or to
    a float32 / float16 numpy array (type and extents taken from it).  ``metadata`` values
    are Python scalars, strings, lists, 1-D numpy arrays or ``Value``s."""
    if version not in VERSIONS:
        raise GGUFError(f"GGUF version {version} is not supported")
    if alignment < 1 or alignment & (alignment - 1):
        raise GGUFError("alignment must be a power of two")
    metadata = dict(metadata or {})
    if alignment != DEFAULT_ALIGNMENT:
        metadata["general.alignment"] = Value(UINT32, alignment)
    head = bytearray(MAGIC + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for key, value in metadata.items():
        value = _infer(value)
        head += _encode(STRING, key) + struct.pack("<I", value.type) + _encode(value.type, value.value,
                                                                              value.element_type)
    blobs, offset = [], 0
    for name, spec in tensors.items():
        if isinstance(spec, np.ndarray):
            codes = {np.dtype(np.float32): 0, np.dtype(np.float16): 1}
            if spec.dtype not in codes:
                raise GGUFError(f"{name}: give (ggml_type, ne, data) for {spec.dtype} tensors")
            spec = (codes[spec.dtype], tuple(reversed(spec.shape)), spec)
        ggml_type, ne, data = spec
        ne = tuple(int(n) for n in ne)
        blob = np.ascontiguousarray(data).view(np.uint8).tobytes()
        if len(blob) != tensor_nbytes(ggml_type, ne):
            raise GGUFError(f"{name}: {len(blob)} bytes given, {tensor_nbytes(ggml_type, ne)} expected")
        head += _encode(STRING, name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        head += struct.pack("<IQ", ggml_type, offset)
        blobs.append((offset, blob))
        offset = -(-(offset + len(blob)) // alignment) * alignment
    data_offset = -(-len(head) // alignment) * alignment
    path = Path(path)
    with open(path, "wb") as handle:
        handle.write(head + bytes(data_offset - len(head)))
        position = 0
        for start, blob in blobs:
            handle.write(bytes(start - position) + blob)
            position = start + len(blob)
    return path
