"""Device buffers and their lifetimes (reference: src/tensor/runtime/buffer.py:11-191).

A Buffer is a contiguous allocation valid within one device session; a
BufferView borrows a base allocation under another contiguous shape.
"""

from __future__ import annotations

import ctypes as c
import math

import numpy as np

from tensor_amd.runtime.abi import DTYPES, BufferDescriptor
from tensor_amd.runtime.errors import TensorRuntimeError


class Buffer:
    """Contiguous owned (or borrowed) device allocation."""

    def __init__(self, device, pointer: int, shape: tuple, dtype, *, owner=None):
        self.device = device
        self._pointer = pointer
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._owner = owner
        self._generation = device._generation
        self.owned = owner is None
        self._nbytes = self._dtype.itemsize * math.prod(self._shape)
        strides, stride = [], self._dtype.itemsize
        for extent in reversed(self._shape):
            strides.insert(0, stride)
            stride *= extent
        self._strides = tuple(strides)
        self._abi_shape = (c.c_int64 * len(self._shape))(*self._shape)
        self._abi_strides = (c.c_int64 * len(strides))(*strides)
        self._descriptor = BufferDescriptor(
            pointer,
            self._nbytes,
            self._abi_shape,
            self._abi_strides,
            len(self._shape),
            DTYPES.get(str(self._dtype), 0),
            device.device_type,
            device.ordinal,
        )
        self._released = False
        self._dlpack_exports = 0

    pointer = property(lambda self: self._pointer)
    shape = property(lambda self: self._shape)
    dtype = property(lambda self: self._dtype)
    nbytes = property(lambda self: self._nbytes)
    strides = property(lambda self: self._strides)

    def __repr__(self):
        state = "released" if self._released else hex(self._pointer)
        return f"Buffer(shape={self._shape}, dtype={self._dtype}, {state})"

    def view(self, shape):
        """Borrow this allocation with another contiguous shape; never copies."""
        return BufferView(self, shape)

    def prefix(self, shape):
        """Borrow a contiguous logical prefix of the allocation."""
        return BufferView(self, shape, prefix=True)

    def copy_from(self, source):
        """Copy equal-sized storage, ordered on the device's stream."""
        self._check()
        source._check()
        if source.device is not self.device:
            raise ValueError("buffer copy requires the same device")
        if source.dtype != self.dtype or source.nbytes != self.nbytes:
            raise ValueError("buffer copy requires the same dtype and storage size")
        self.device._copy(self, source)
        return self

    def copy_columns_from(self, source, offset=0):
        """``self[:, offset:offset + source.shape[1]] = source`` on the device."""
        self._check()
        source._check()
        if source.device is not self.device:
            raise ValueError("buffer copy requires the same device")
        if self.dtype != source.dtype or len(self.shape) != 2 or len(source.shape) != 2:
            raise ValueError("column copy requires two matrices with the same dtype")
        if (self.shape[0] != source.shape[0] or type(offset) is not int or offset < 0
                or offset + source.shape[1] > self.shape[1]):
            raise ValueError("column copy exceeds matrix rows or columns")
        self.device._copy_columns(self, source, offset)
        return self

    def _check(self) -> None:
        self.device._check()
        if self._generation != self.device._generation:
            raise self.device.error("buffer belongs to a previous device session")
        if self._released:
            raise self.device.error("buffer has been released")

    def to_numpy(self):
        self._check()
        self.device.synchronize()
        return self.device._download(self)

    def to_bytes(self) -> bytes:
        return self.to_numpy().tobytes()

    def release(self) -> None:
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
        self._released = True
        self.device._buffers.discard(self)

    def __dlpack_device__(self):
        self._check()
        return self.device.device_type, self.device.ordinal

    def __dlpack__(self, *, stream=None, max_version=None, dl_device=None, copy=None):
        export = getattr(self.device, "_export_dlpack", None)
        if export is None:
            raise BufferError("DLPack export is not provided by this provider")
        return export(self, stream=stream, max_version=max_version, dl_device=dl_device, copy=copy)


class BufferView(Buffer):
    """A reshape descriptor borrowing storage and lifetime from another buffer."""

    def __init__(self, base, shape, *, prefix=False):
        base._check()
        shape = (shape,) if type(shape) is int else tuple(shape)
        if not shape or any(type(n) is not int or n < 1 for n in shape):
            raise ValueError("view shape must contain positive integers")
        size = math.prod(shape) * base.dtype.itemsize
        if prefix and size > base.nbytes:
            raise ValueError("logical prefix exceeds buffer capacity")
        if not prefix and size != base.nbytes:
            raise ValueError("reshape view must preserve buffer storage size")
        super().__init__(base.device, base._pointer, shape, base.dtype, owner=base)
        self._base = base
        self.device._buffers.add(self)

    def _check(self):
        super()._check()
        self._base._check()

    def release(self):
        if not self._released:
            self.device._check()
            self.device.synchronize()
            self._dispose()

    def _dispose(self):
        if self._released:
            return
        if self._dlpack_exports:
            raise TensorRuntimeError("release DLPack consumers before releasing this buffer")
        self._released = True
        self.device._buffers.discard(self)
