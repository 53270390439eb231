"""kDLROCM DLPack exchange (tensor_amd.runtime.dlpack), checked on the CPU.

Synthetic producers hand out capsules over fake device pointers: nothing here
dereferences device memory.  Mirrors the capsule rules the reference relies on
(src/tensor/runtime/dlpack.py): a consumed capsule is renamed ``used_...`` and
its deleter runs exactly once, also when the import is refused.
"""

from __future__ import annotations

import ctypes as c
import gc
from types import SimpleNamespace

import numpy as np
import pytest

from tensor_amd.runtime import dlpack as D
from tensor_amd.runtime.buffer import Buffer


def test_struct_layouts_match_the_dlpack_abi():
    assert [c.sizeof(s) for s in (D.DLDevice, D.DLDataType, D.DLTensor, D.DLManagedTensor,
                                  D.DLManagedTensorVersioned)] == [8, 4, 48, 64, 80]
    assert D.DLManagedTensorVersioned.dl_tensor.offset == 32 and D.DLManagedTensor.deleter.offset == 56


class Producer:
    """A DLPack producer over a fake pointer; counts deleter calls and remembers the stream."""

    def __init__(self, shape=(4, 8), dtype=(2, 16), device=(10, 0), data=0x10000, strides=None, offset=0,
                 flags=0, versioned=True, major=1, keyword=True):
        self.deleted, self.stream, self.capsule = 0, "unset", None
        self._shape = (c.c_int64 * len(shape))(*shape)
        self._strides = (c.c_int64 * len(strides))(*strides) if strides else None
        tensor = D.DLTensor(data, D.DLDevice(*device), len(shape), D.DLDataType(dtype[0], dtype[1], 1),
                            self._shape, self._strides, offset)

        @D._DELETER
        def deleter(address):
            self.deleted += 1

        self._deleter = deleter
        pointer = c.cast(deleter, c.c_void_p)
        if versioned:
            self.managed = D.DLManagedTensorVersioned(D.DLPackVersion(major, 0), None, pointer, flags, tensor)
        else:
            self.managed = D.DLManagedTensor(tensor, None, pointer)
        self.name = b"dltensor_versioned" if versioned else b"dltensor"
        self.keyword = keyword

    def _capsule(self, stream):
        self.stream = stream
        self.capsule = D._new_capsule(c.addressof(self.managed), self.name, None)
        return self.capsule

    def __dlpack__(self, stream=None, **kwargs):
        if not self.keyword and "max_version" in kwargs:
            raise TypeError("__dlpack__() got an unexpected keyword argument 'max_version'")
        return self._capsule(stream)

    def __dlpack_device__(self):
        return tuple(self.managed.dl_tensor.device.device_type, ) + (self.managed.dl_tensor.device.device_id,)


def test_borrow_reads_the_tensor_and_releases_once():
    producer = Producer(offset=64)
    owner, address, shape, dtype = D.borrow(producer, stream=7, device_type=D.KDL_ROCM, ordinal=0)
    assert (address, shape, dtype) == (0x10000 + 64, (4, 8), np.dtype(np.float16))
    assert producer.stream == 7
    assert D._get_name(producer.capsule) == b"used_dltensor_versioned"
    assert producer.deleted == 0
    owner.release()
    owner.release()
    assert producer.deleted == 1


def test_legacy_capsules_and_producers_without_max_version():
    producer = Producer(versioned=False, keyword=False, dtype=(1, 8), shape=(3,))
    owner, address, shape, dtype = D.borrow(producer, stream=0, device_type=D.KDL_ROCM, ordinal=0)
    assert (shape, dtype) == ((3,), np.dtype(np.uint8))
    assert D._get_name(producer.capsule) == b"used_dltensor"
    owner.release()
    assert producer.deleted == 1


def test_compact_strides_are_accepted():
    producer = Producer(shape=(4, 8), strides=(8, 1))
    owner, *_ = D.borrow(producer, stream=0, device_type=D.KDL_ROCM, ordinal=0)
    owner.release()
    # a size-1 axis may carry any stride
    producer = Producer(shape=(1, 8), strides=(123, 1))
    owner, *_ = D.borrow(producer, stream=0, device_type=D.KDL_ROCM, ordinal=0)
    owner.release()


@pytest.mark.parametrize("kwargs,needle", [
    ({"device": (2, 0)}, "device"),                   # a CUDA tensor
    ({"device": (10, 1)}, "device"),                  # another ROCm device
    ({"flags": D.READ_ONLY}, "read-only"),
    ({"flags": 1 << 7}, "flags"),
    ({"major": 2}, "major version"),
    ({"strides": (1, 4)}, "row-major"),               # column-major
    ({"dtype": (4, 16)}, "element type"),             # bfloat16 has no numpy dtype
    ({"dtype": (2, 8)}, "element type"),
    ({"data": 0}, "null"),
    ({"data": 0x10001}, "misaligned"),
    ({"shape": (4, 0)}, "positive"),
])
def test_refused_imports_still_release_the_producer(kwargs, needle):
    producer = Producer(**kwargs)
    with pytest.raises(BufferError, match=needle):
        D.borrow(producer, stream=0, device_type=D.KDL_ROCM, ordinal=0)
    assert producer.deleted == 1


def test_a_consumed_capsule_is_refused():
    producer = Producer()
    capsule = producer.__dlpack__(stream=0)
    D.ImportedTensor(capsule, producer).release()
    with pytest.raises(BufferError, match="unconsumed"):
        D.ImportedTensor(capsule, producer)
    assert producer.deleted == 1


def fake_buffer(shape=(2, 3), dtype=np.float32, pointer=0x20000, ordinal=3):
    device = SimpleNamespace(device_type=D.KDL_ROCM, ordinal=ordinal, _generation=0)
    return Buffer(device, pointer, shape, dtype)


@pytest.mark.parametrize("versioned", [True, False])
def test_export_round_trip_holds_the_buffer_until_the_deleter(versioned):
    buffer = fake_buffer()
    capsule = D.export(buffer, device_type=D.KDL_ROCM, versioned=versioned)
    assert buffer._dlpack_exports == 1
    owner = D.ImportedTensor(capsule, buffer)
    assert owner.describe(D.KDL_ROCM, 3) == (0x20000, (2, 3), np.dtype(np.float32))
    assert owner.managed.dl_tensor.strides is None or not owner.managed.dl_tensor.strides
    del capsule
    gc.collect()
    assert buffer._dlpack_exports == 1  # consumed: only the consumer's deleter call releases it
    owner.release()
    assert buffer._dlpack_exports == 0


def test_an_unconsumed_export_releases_on_capsule_destruction():
    buffer = fake_buffer(shape=(5,), dtype=np.uint8)
    capsule = D.export(buffer, device_type=D.KDL_ROCM, versioned=True)
    assert buffer._dlpack_exports == 1
    del capsule
    gc.collect()
    assert buffer._dlpack_exports == 0 and not D._exports


def test_export_dtype_codes():
    assert (D.dlpack_dtype(np.float16).code, D.dlpack_dtype(np.float16).bits) == (2, 16)
    assert (D.dlpack_dtype(np.uint8).code, D.dlpack_dtype(np.int32).code, D.dlpack_dtype(np.bool_).code) == (1, 0, 6)
    with pytest.raises(BufferError):
        D.dlpack_dtype(np.complex64)


def test_buffer_export_needs_provider_support():
    with pytest.raises(BufferError, match="not provided"):
        fake_buffer().__dlpack__()

