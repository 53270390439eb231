"""DLPack exchange of device buffers with kDLROCM (device type 10).

The reference's runtime imports and exports DLPack capsules for CUDA only: both
paths fix device type 2 (src/tensor/runtime/dlpack.py:103, :210).  This module
is the ROCm counterpart.  The structures are the public DLPack ABI
(https://dmlc.github.io/dlpack/latest/: DLDevice, DLDataType, DLTensor,
DLManagedTensor and, from DLPack 1.0, DLManagedTensorVersioned); the capsule
rules are the Python specification's: a producer hands out a capsule named
``dltensor`` (or ``dltensor_versioned``), a consumer renames it ``used_...``
and from then on owns the single call of the deleter; a capsule destroyed
without having been consumed calls the deleter itself.  No producer framework
is imported here.
"""

from __future__ import annotations

import ctypes as c

import numpy as np

KDL_CPU = 1
KDL_ROCM = 10
READ_ONLY = 1 << 0  # DLPACK_FLAG_BITMASK_READ_ONLY
IS_COPIED = 1 << 1  # DLPACK_FLAG_BITMASK_IS_COPIED


class DLDevice(c.Structure):
    _fields_ = [("device_type", c.c_int32), ("device_id", c.c_int32)]


class DLDataType(c.Structure):
    _fields_ = [("code", c.c_uint8), ("bits", c.c_uint8), ("lanes", c.c_uint16)]


class DLTensor(c.Structure):
    _fields_ = [
        ("data", c.c_void_p),
        ("device", DLDevice),
        ("ndim", c.c_int32),
        ("dtype", DLDataType),
        ("shape", c.POINTER(c.c_int64)),
        ("strides", c.POINTER(c.c_int64)),
        ("byte_offset", c.c_uint64),
    ]


class DLManagedTensor(c.Structure):
    _fields_ = [("dl_tensor", DLTensor), ("manager_ctx", c.c_void_p), ("deleter", c.c_void_p)]


class DLPackVersion(c.Structure):
    _fields_ = [("major", c.c_uint32), ("minor", c.c_uint32)]


class DLManagedTensorVersioned(c.Structure):
    _fields_ = [
        ("version", DLPackVersion),
        ("manager_ctx", c.c_void_p),
        ("deleter", c.c_void_p),
        ("flags", c.c_uint64),
        ("dl_tensor", DLTensor),
    ]


# DLDataType codes: kDLInt 0, kDLUInt 1, kDLFloat 2, kDLBool 6 (kDLBfloat 4 has no numpy dtype)
_KIND_TO_CODE = {"i": 0, "u": 1, "f": 2, "b": 6}
_CODE_TO_KIND = {0: "int", 1: "uint", 2: "float"}

_api = c.pythonapi
_get_name = _api.PyCapsule_GetName
_get_name.argtypes, _get_name.restype = [c.py_object], c.c_char_p
_get_pointer = _api.PyCapsule_GetPointer
_get_pointer.argtypes, _get_pointer.restype = [c.py_object, c.c_char_p], c.c_void_p
_set_name = _api.PyCapsule_SetName
_set_name.argtypes, _set_name.restype = [c.py_object, c.c_char_p], c.c_int
_new_capsule = _api.PyCapsule_New
_new_capsule.argtypes, _new_capsule.restype = [c.c_void_p, c.c_char_p, c.c_void_p], c.py_object
# PyCapsule keeps a pointer to its name: these bytes objects live as long as the module.
_CONSUMED = {b"dltensor": b"used_dltensor", b"dltensor_versioned": b"used_dltensor_versioned"}
_DELETER = c.CFUNCTYPE(None, c.c_void_p)


def numpy_dtype(dtype: DLDataType) -> np.dtype:
    """The numpy dtype of a single-lane DLPack element type."""
    if dtype.lanes != 1:
        raise BufferError("vector (multi-lane) DLPack dtypes are not supported")
    if dtype.code == 6 and dtype.bits == 8:
        return np.dtype(np.bool_)
    if dtype.code == 2 and dtype.bits in (16, 32, 64):
        return np.dtype(f"float{dtype.bits}")
    if dtype.code in (0, 1) and dtype.bits in (8, 16, 32, 64):
        return np.dtype(f"{_CODE_TO_KIND[dtype.code]}{dtype.bits}")
    raise BufferError(f"unsupported DLPack element type (code {dtype.code}, {dtype.bits} bits)")


def dlpack_dtype(dtype) -> DLDataType:
    dtype = np.dtype(dtype)
    if dtype.kind not in _KIND_TO_CODE:
        raise BufferError(f"dtype {dtype} has no DLPack element type")
    return DLDataType(_KIND_TO_CODE[dtype.kind], dtype.itemsize * 8, 1)


class ImportedTensor:
    """A consumed DLPack capsule: the producer's memory, held until release()."""

    def __init__(self, capsule, source):
        name = _get_name(capsule)
        if name not in _CONSUMED:
            raise BufferError("expected an unconsumed 'dltensor' or 'dltensor_versioned' capsule")
        self.address = _get_pointer(capsule, name)
        if not self.address:
            raise BufferError("DLPack capsule holds a null managed tensor")
        self.versioned = name == b"dltensor_versioned"
        kind = DLManagedTensorVersioned if self.versioned else DLManagedTensor
        self.managed = c.cast(self.address, c.POINTER(kind)).contents
        # from here on the deleter is ours to call, exactly once
        _set_name(capsule, _CONSUMED[name])
        self._capsule, self._source, self._released = capsule, source, False

    def describe(self, device_type: int, ordinal: int):
        """(address, shape, dtype) of a contiguous tensor on the given device; BufferError otherwise."""
        if self.versioned:
            if self.managed.version.major != 1:
                raise BufferError(f"unsupported DLPack major version {self.managed.version.major}")
            if self.managed.flags & READ_ONLY:
                raise BufferError("read-only DLPack tensors cannot be bound to kernels that write")
            if self.managed.flags & ~(READ_ONLY | IS_COPIED):
                raise BufferError("unknown DLPack flags")
        tensor = self.managed.dl_tensor
        if tensor.device.device_type != device_type or tensor.device.device_id != ordinal:
            raise BufferError(f"DLPack tensor is on device ({tensor.device.device_type}, {tensor.device.device_id}), "
                              f"not ({device_type}, {ordinal})")
        if not 1 <= tensor.ndim <= 64 or not tensor.shape:
            raise BufferError("DLPack tensor needs 1 to 64 dimensions")
        shape = tuple(int(tensor.shape[i]) for i in range(tensor.ndim))
        if any(extent < 1 for extent in shape):
            raise BufferError("DLPack tensor needs positive extents")
        dtype = numpy_dtype(tensor.dtype)
        if tensor.strides:  # element strides; NULL means compact row-major
            expected = 1
            for axis in reversed(range(tensor.ndim)):
                if shape[axis] > 1 and tensor.strides[axis] != expected:
                    raise BufferError("only compact row-major DLPack tensors can be imported")
                expected *= shape[axis]
        address = (tensor.data or 0) + tensor.byte_offset
        if not tensor.data or address >= 1 << 64 or address % dtype.itemsize:
            raise BufferError("null or misaligned DLPack data pointer")
        return address, shape, dtype

    def release(self) -> None:
        if self._released:
            return
        self._released = True
        deleter = self.managed.deleter
        if deleter:
            _DELETER(deleter)(self.address)
        self._capsule = self._source = self.managed = None


def borrow(source, *, stream, device_type: int, ordinal: int):
    """Consume ``source.__dlpack__(stream=stream)``: (owner, address, shape, dtype).
    The producer orders its pending writes before ``stream`` (DLPack's stream rule)."""
    try:
        capsule = source.__dlpack__(stream=stream, max_version=(1, 0))
    except TypeError as exc:
        if "max_version" not in str(exc):
            raise
        capsule = source.__dlpack__(stream=stream)
    owner = ImportedTensor(capsule, source)
    try:
        address, shape, dtype = owner.describe(device_type, ordinal)
    except BaseException:
        owner.release()
        raise
    return owner, address, shape, dtype


# -------------------------------------------------------------------- export --
# Each export keeps its structures and the exporting buffer (and the buffers it views)
# alive until the consumer calls the deleter, or until an unconsumed capsule is destroyed.
_exports: dict = {}


# The capsule destructor receives the capsule while it is being deallocated: it must not
# take a Python reference to it, so it reads the capsule through these void* entry points.
_raw_get_name = c.PYFUNCTYPE(c.c_char_p, c.c_void_p)(("PyCapsule_GetName", _api))
_raw_get_pointer = c.PYFUNCTYPE(c.c_void_p, c.c_void_p, c.c_char_p)(("PyCapsule_GetPointer", _api))


def _release_export(address) -> None:
    record = _exports.pop(address, None)
    if record is not None:
        for buffer in record[2]:
            buffer._dlpack_exports -= 1


@_DELETER
def _delete_export(address):
    _release_export(address)


@_DELETER
def _destroy_capsule(capsule):
    name = _raw_get_name(capsule)
    if name in _CONSUMED:  # never consumed: the producer still owns the deleter call
        _release_export(_raw_get_pointer(capsule, name))


def export(buffer, *, device_type: int, versioned: bool):
    """A capsule describing ``buffer`` (compact row-major, NULL strides) on its device."""
    shape = (c.c_int64 * len(buffer.shape))(*buffer.shape)
    tensor = DLTensor(buffer.pointer, DLDevice(device_type, buffer.device.ordinal), len(buffer.shape),
                      dlpack_dtype(buffer.dtype), shape, None, 0)
    deleter = c.cast(_delete_export, c.c_void_p)
    if versioned:
        managed = DLManagedTensorVersioned(DLPackVersion(1, 0), None, deleter, 0, tensor)
    else:
        managed = DLManagedTensor(tensor, None, deleter)
    address = c.addressof(managed)
    holders = [buffer]
    while getattr(holders[-1], "_base", None) is not None:
        holders.append(holders[-1]._base)
    for holder in holders:
        holder._dlpack_exports += 1
    _exports[address] = (managed, shape, holders)
    try:
        return _new_capsule(address, b"dltensor_versioned" if versioned else b"dltensor",
                            c.cast(_destroy_capsule, c.c_void_p))
    except BaseException:
        _release_export(address)
        raise
