"""Device buffers (the reference's Buffer / BufferView surface, src/tensor/runtime/buffer.py).

A ``Buffer`` is a contiguous row-major view of one ``_Storage``: the device address range an
allocation (or a borrowed DLPack producer) provides, its owner and whether it is still live.
Views made with ``view`` or ``prefix`` share their base's storage record, so releasing the
base invalidates every view at once, and releasing a view never frees the memory.  Each
buffer builds its TensorBufferV1 descriptor once and keeps the shape and stride arrays it
points to alive with it.
"""

from __future__ import annotations

import ctypes as c
import math

import numpy as np

from tensor_amd.runtime.abi import DTYPES, BufferDescriptor
from tensor_amd.runtime.errors import TensorRuntimeError


class _Storage:
    """A device address range and its lifetime, shared by a buffer and its views."""

    __slots__ = ("address", "capacity", "owner", "live", "generation")

    def __init__(self, address: int, capacity: int, owner, generation: int):
        self.address, self.capacity, self.owner = address, capacity, owner
        self.live, self.generation = True, generation


def _contiguous_strides(shape: tuple, itemsize: int) -> tuple:
    strides = [itemsize] * len(shape)
    for axis in range(len(shape) - 2, -1, -1):
        strides[axis] = strides[axis + 1] * shape[axis + 1]
    return tuple(strides)


class Buffer:
    """A contiguous device buffer valid inside one device session."""

    def __init__(self, device, pointer: int, shape: tuple, dtype, *, owner=None, _storage=None):
        self.device = device
        self._shape = tuple(int(n) for n in shape)
        self._dtype = np.dtype(dtype)
        self._nbytes = self._dtype.itemsize * math.prod(self._shape)
        self._storage = _storage or _Storage(pointer, self._nbytes, owner, device._generation)
        self._base = None
        self._dlpack_exports = 0
        self._own_live = True
        strides = _contiguous_strides(self._shape, self._dtype.itemsize)
        self._strides = strides
        self._abi_arrays = ((c.c_int64 * len(self._shape))(*self._shape), (c.c_int64 * len(strides))(*strides))
        self._descriptor = BufferDescriptor(pointer, self._nbytes, self._abi_arrays[0], self._abi_arrays[1],
                                            len(self._shape), DTYPES.get(self._dtype.name, 0), device.device_type,
                                            device.ordinal)

    # -- read-only properties ------------------------------------------------
    pointer = property(lambda self: self._storage.address)
    shape = property(lambda self: self._shape)
    dtype = property(lambda self: self._dtype)
    nbytes = property(lambda self: self._nbytes)
    strides = property(lambda self: self._strides)
    owned = property(lambda self: self._base is None and self._storage.owner is None)
    _owner = property(lambda self: self._storage.owner)
    _generation = property(lambda self: self._storage.generation)

    @property
    def _released(self) -> bool:
        return not (self._own_live and self._storage.live)

    def __repr__(self):
        where = "released" if self._released else hex(self.pointer)
        return f"Buffer(shape={self._shape}, dtype={self._dtype}, {where})"

    # -- lifetime -------------------------------------------------------------
    def _check(self) -> None:
        self.device._check()
        if self._storage.generation != self.device._generation:
            raise self.device.error("buffer belongs to a previous device session")
        if self._released:
            raise self.device.error("buffer has been released")

    def release(self) -> None:
        """Wait for the device, then free the memory (or hand a borrowed producer back)."""
        if not self._released:
            self._check()
            self.device.synchronize()
            self._dispose()

    def _dispose(self) -> None:
        if self._released:
            return
        if self._dlpack_exports:
            raise TensorRuntimeError("release DLPack consumers before releasing this buffer")
        self.device._dispose_buffer(self)
        self._storage.owner = None
        self._storage.live = False
        self.device._buffers.discard(self)

    # -- views and copies -----------------------------------------------------
    def view(self, shape):
        """The same storage under another contiguous shape of equal size."""
        return BufferView(self, shape)

    def prefix(self, shape):
        """The leading bytes of the storage under a (smaller or equal) contiguous shape."""
        return BufferView(self, shape, prefix=True)

    def copy_from(self, source):
        """Copy equal-sized storage from another buffer of this device, ordered on its stream."""
        self._check()
        source._check()
        if source.device is not self.device:
            raise ValueError("buffer copy requires the same device")
        if (source.dtype, source.nbytes) != (self.dtype, self.nbytes):
            raise ValueError("buffer copy requires the same dtype and storage size")
        self.device._copy(self, source)
        return self

    def copy_columns_from(self, source, offset=0):
        """``self[:, offset:offset + source.shape[1]] = source`` for two matrices on the device."""
        self._check()
        source._check()
        if source.device is not self.device:
            raise ValueError("buffer copy requires the same device")
        if len(self.shape) != 2 or len(source.shape) != 2 or self.dtype != source.dtype:
            raise ValueError("column copy requires two matrices with the same dtype")
        if type(offset) is not int or offset < 0 or source.shape[0] != self.shape[0] \
                or offset + source.shape[1] > self.shape[1]:
            raise ValueError("column copy exceeds matrix rows or columns")
        self.device._copy_columns(self, source, offset)
        return self

    def to_numpy(self):
        self._check()
        self.device.synchronize()
        return self.device._download(self)

    def to_bytes(self) -> bytes:
        return self.to_numpy().tobytes()

    # -- DLPack ---------------------------------------------------------------
    def __dlpack_device__(self):
        self._check()
        return self.device.device_type, self.device.ordinal

    def __dlpack__(self, *, stream=None, max_version=None, dl_device=None, copy=None):
        exporter = getattr(self.device, "_export_dlpack", None)
        if exporter is None:
            raise BufferError("DLPack export is not provided by this provider")
        return exporter(self, stream=stream, max_version=max_version, dl_device=dl_device, copy=copy)


class BufferView(Buffer):
    """Another contiguous shape over a base buffer's storage; it never owns memory."""

    def __init__(self, base: Buffer, shape, *, prefix: bool = False):
        base._check()
        shape = (shape,) if type(shape) is int else tuple(shape)
        if not shape or any(type(n) is not int or n < 1 for n in shape):
            raise ValueError("view shape must contain positive integers")
        nbytes = math.prod(shape) * base.dtype.itemsize
        if nbytes > base.nbytes if prefix else nbytes != base.nbytes:
            raise ValueError("logical prefix exceeds buffer capacity" if prefix
                             else "reshape view must preserve buffer storage size")
        super().__init__(base.device, base.pointer, shape, base.dtype, _storage=base._storage)
        self._base = base
        self.device._buffers.add(self)

    def _check(self) -> None:
        super()._check()
        self._base._check()

    def release(self) -> None:
        if not self._released:
            self.device._check()
            self.device.synchronize()
            self._dispose()

    def _dispose(self) -> None:
        if self._released:
            return
        if self._dlpack_exports:
            raise TensorRuntimeError("release DLPack consumers before releasing this buffer")
        self._own_live = False
        self.device._buffers.discard(self)
