"""ROCm/HIP runtime provider for one MI355X (gfx950) device.

Behavioural template: the reference CUDA provider
(src/tensor/providers/cuda/device.py:16-448) — a session owns (or borrows) a
stream, allocates buffers, loads executables, launches them asynchronously
through the TensorCallV1 descriptor and records events.  Every device call goes
through libtensor_hip.so (include/tensor_hip.h): the kernels are its
TensorKernelV1 entry points and memory/streams/events are its runtime services.

Executables are the library's built-in GGUF kernels, loaded by name
(``device.load("gguf_linear", encoding="q4_k")``) or from a manifest dict.
"""

from __future__ import annotations

import contextlib
import ctypes as c
import threading

import numpy as np

from tensor_amd import _native
from tensor_amd._native import HipError, TensorHipDeviceInfo
from tensor_amd.runtime.abi import CAPABILITIES, DEVICE_ROCM, ErrorDescriptor, StreamDescriptor, check_requirement
from tensor_amd.runtime.buffer import Buffer
from tensor_amd.runtime.event import Event
from tensor_amd.runtime.executable import Executable
from tensor_amd.runtime.session import Session

# Multi-row Q4_K GEMV kernels by plan index, and the launch fields (a, b) each accepts:
# sector-aligned tiles (tiles per workgroup, x staged before the weight loads), multi-tile with x
# in LDS (tiles per workgroup, super-blocks per wave), x read per wave (waves splitting K, 0).
GEMV_KERNELS = ("sec", "mt", "mfma", "sec_split")
GEMV_FIELDS = {0: [(a, b) for a in (1, 2, 3) for b in (0, 1)],
               1: [(a, b) for a in (1, 2) for b in (2, 3)],
               2: [(4, 0), (8, 0)],
               3: [(a, b) for a in (1, 2, 3, 4, 5, 6, 8) for b in (2, 4)]}


def gemm_tiles() -> list:
    """Every tile of the pipelined prefill GEMM, by index: {"bm", "bn", "ks"}."""
    tiles = []
    while True:
        bm, bn, ks = c.c_int32(), c.c_int32(), c.c_int32()
        error = ErrorDescriptor()
        if _native.library().tensor_gguf_gemm_tile_v1(len(tiles), c.byref(bm), c.byref(bn), c.byref(ks),
                                                       c.byref(error)):
            return tiles
        tiles.append({"bm": bm.value, "bn": bn.value, "ks": ks.value})


# The device this library last made current on each thread (HIP's current device is per thread).
# Launches consult it instead of setting the device again; an entry point that finds another
# current device (set by other code on the thread) refuses the call before enqueuing anything,
# and the launch then sets the device and submits once more.
_thread = threading.local()
_NOT_CURRENT = b"is not the current device"


def device_count() -> int:
    count = c.c_int32()
    _native.call("tensor_hip_device_count", c.byref(count))
    return count.value


class Device(Session):
    device_type = DEVICE_ROCM
    error = HipError
    capabilities = CAPABILITIES | {"events", "async_launch", "external_streams", "graphs"}

    def __init__(self, ordinal: int = 0, *, stream: int | None = None):
        if type(ordinal) is not int or ordinal < 0:
            raise ValueError("ordinal must be a non-negative integer")
        if stream is not None and (type(stream) is not int or not 0 <= stream < 1 << 64):
            raise ValueError("stream must be a HIP stream integer handle")
        self.ordinal = ordinal
        self._external_stream = stream
        self.owns_stream = stream is None
        count = device_count()
        if ordinal >= count:
            raise ValueError(f"HIP device {ordinal} is not present ({count} visible)")
        props = TensorHipDeviceInfo()
        _native.call("tensor_hip_device_info", ordinal, c.byref(props))
        arch = props.arch.decode()
        self.info = {
            "ordinal": ordinal,
            "name": props.name.decode(),
            "arch": arch.split(":")[0],
            "arch_features": arch,
            "provider": "hip",
            "compute_units": props.compute_units,
            "clock_khz": props.clock_khz,
            "memory_clock_khz": props.memory_clock_khz,
            "memory_bus_width": props.memory_bus_width,
            "total_memory": props.total_memory,
            "l2_cache_bytes": props.l2_cache_bytes,
            "warp_size": props.warp_size,
        }
        self.limits = {
            "grid": list(props.max_grid),
            "block": list(props.max_block),
            "threads": props.max_threads_per_block,
            "shared_memory_bytes": props.max_shared_memory_per_block,
        }
        self.stream = 0
        self._buffers: set = set()
        self._consumers: set = set()
        self._graphs: set = set()
        self._capture_log = None  # list of buffers while a HipGraph capture is open
        self._generation = 0
        self._open = False

    # ------------------------------------------------------------ session --
    def __enter__(self) -> "Device":
        if self._open:
            raise HipError("Device", 3, "device session is already open")
        _native.call("tensor_hip_set_device", self.ordinal)
        if self.owns_stream:
            handle = c.c_uint64()
            _native.call("tensor_hip_stream_create", c.byref(handle))
            self.stream = handle.value
        else:
            self.stream = self._external_stream
        self._generation += 1
        self._start_session()
        self._open = True
        return self

    def _check(self) -> None:
        if not self._open:
            raise HipError("Device", 3, "HIP device session is closed")
        _native.call("tensor_hip_set_device", self.ordinal)
        _thread.ordinal = self.ordinal

    def _make_current(self) -> None:
        """The launch path's device check: no native call when this thread's device is set."""
        if not self._open:
            raise HipError("Device", 3, "HIP device session is closed")
        if getattr(_thread, "ordinal", None) != self.ordinal:
            _native.call("tensor_hip_set_device", self.ordinal)
            _thread.ordinal = self.ordinal

    def stream_descriptor(self) -> StreamDescriptor:
        return StreamDescriptor(DEVICE_ROCM, self.ordinal, self.stream)

    def synchronize(self) -> None:
        self._check()
        _native.call("tensor_hip_stream_synchronize", self.stream)
        for handle in self._consumers:
            _native.call("tensor_hip_stream_synchronize", handle)

    def _order_streams(self, producer: int, consumer: int) -> None:
        if producer == consumer:
            return
        event = c.c_uint64()
        _native.call("tensor_hip_event_create", c.byref(event), 0)
        try:
            _native.call("tensor_hip_event_record", event.value, producer)
            _native.call("tensor_hip_stream_wait_event", consumer, event.value)
        finally:
            _native.call("tensor_hip_event_destroy", event.value)

    def wait_for(self, producer_stream: int) -> None:
        """Order this session's stream after work queued on another stream."""
        self._check()
        self._order_streams(int(producer_stream), self.stream)

    def handoff(self, consumer_stream: int) -> None:
        """Order another stream after work already queued on this session's stream."""
        self._check()
        self._order_streams(self.stream, int(consumer_stream))
        self._consumers.add(int(consumer_stream))

    # ------------------------------------------------------------ buffers --
    def empty(self, shape, dtype="float32") -> Buffer:
        self._check()
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        if not shape or any(type(size) is not int or size < 1 for size in shape):
            raise ValueError("buffer shape must contain positive integers")
        dtype = np.dtype(dtype)
        if dtype.hasobject or dtype.itemsize < 1:
            raise ValueError("buffer dtype must have a fixed byte size")
        nbytes = dtype.itemsize
        for extent in shape:
            nbytes *= extent
        address = c.c_uint64()
        _native.call("tensor_hip_malloc", nbytes, c.byref(address))
        buffer = Buffer(self, address.value, shape, dtype)
        self._buffers.add(buffer)
        return buffer

    def from_numpy(self, array, dtype=None) -> Buffer:
        host = np.ascontiguousarray(array, dtype=dtype)
        buffer = self.empty(host.shape if host.shape else (1,), host.dtype)
        try:
            _native.call("tensor_hip_copy_htod", buffer.pointer, host.ctypes.data, host.nbytes, self.stream)
            return buffer
        except BaseException:
            buffer.release()
            raise

    def from_dlpack(self, source, *, stream: int | None = None) -> Buffer:
        """Import a DLPack producer (reference: src/tensor/providers/cuda/device.py:278-314 for
        CUDA).  CPU tensors are copied in; ROCm tensors on this device (kDLROCM, 10) are
        borrowed without a copy and keep the producer's memory alive until released.  The
        producer orders its pending writes before ``stream`` (default: this session's)."""
        from tensor_amd.runtime import dlpack

        self._check()
        if not hasattr(source, "__dlpack_device__") or not hasattr(source, "__dlpack__"):
            raise TypeError("DLPack source must implement __dlpack__ and __dlpack_device__")
        kind, ordinal = source.__dlpack_device__()
        if kind == dlpack.KDL_CPU:
            return self.from_numpy(np.from_dlpack(source))
        if kind != dlpack.KDL_ROCM or ordinal != self.ordinal:
            raise BufferError(f"DLPack source must be on the CPU or ROCm device {self.ordinal}")
        owner, address, shape, dtype = dlpack.borrow(source, stream=self.stream if stream is None else int(stream),
                                                     device_type=dlpack.KDL_ROCM, ordinal=self.ordinal)
        try:
            owning, device_memory = c.c_int32(), c.c_int32()
            try:
                _native.call("tensor_hip_pointer_device", address, c.byref(owning), c.byref(device_memory))
            except HipError as exc:
                raise BufferError(f"DLPack pointer is unknown to this HIP runtime ({exc}); a second HIP "
                                  "runtime in the process would explain it") from None
            if not device_memory.value or owning.value != self.ordinal:
                raise BufferError(f"DLPack pointer is not device memory of ROCm device {self.ordinal}")
            buffer = Buffer(self, address, shape, dtype, owner=owner)
            self._buffers.add(buffer)
            return buffer
        except BaseException:
            owner.release()
            raise

    def _export_dlpack(self, buffer: Buffer, *, stream=None, max_version=None, dl_device=None, copy=None):
        """Buffer.__dlpack__: a kDLROCM capsule of the buffer, after this session's queued work
        has been ordered before the consumer's ``stream`` (None: the null stream, -1: no ordering)."""
        from tensor_amd.runtime import dlpack

        buffer._check()
        if copy:
            raise BufferError("DLPack export shares the buffer; copy=True is not supported")
        if dl_device is not None and tuple(dl_device) != (DEVICE_ROCM, self.ordinal):
            raise BufferError("DLPack export is only to this ROCm device")
        consumer = 0 if stream is None else int(stream)
        if consumer != -1:
            self.handoff(consumer)
        versioned = max_version is not None and int(max_version[0]) >= 1
        return dlpack.export(buffer, device_type=DEVICE_ROCM, versioned=versioned)

    def upload(self, buffer: Buffer, array) -> Buffer:
        """Overwrite a buffer's contents from host memory (synchronous)."""
        buffer._check()
        host = np.ascontiguousarray(array, dtype=buffer.dtype)
        if host.nbytes != buffer.nbytes:
            raise ValueError("upload needs exactly the buffer's storage size")
        _native.call("tensor_hip_copy_htod", buffer.pointer, host.ctypes.data, host.nbytes, self.stream)
        return buffer

    def full(self, shape, fill_value, dtype="float32") -> Buffer:
        return self.from_numpy(np.full(shape, fill_value, dtype=dtype))

    def zeros(self, shape, dtype="float32") -> Buffer:
        buffer = self.empty(shape, dtype)
        try:
            _native.call("tensor_hip_fill_u8", buffer.pointer, 0, buffer.nbytes, self.stream)
            return buffer
        except BaseException:
            buffer.release()
            raise

    def ones(self, shape, dtype="float32") -> Buffer:
        return self.full(shape, 1, dtype)

    def randn(self, shape, dtype="float32", *, seed=None) -> Buffer:
        return self.from_numpy(np.random.default_rng(seed).standard_normal(shape).astype(dtype))

    def arange(self, stop: int, dtype="float32") -> Buffer:
        return self.from_numpy(np.arange(stop, dtype=dtype))

    def fill_bytes(self, buffer: Buffer, value: int) -> None:
        """Set every byte of a buffer (ordered on the stream)."""
        buffer._check()
        _native.call("tensor_hip_fill_u8", buffer.pointer, int(value) & 0xFF, buffer.nbytes, self.stream)

    def _download_storage(self, buffer) -> np.ndarray:
        """The buffer's bytes on the host as an array of its storage dtype, after the work
        queued on this stream: the hook the reference's ``Buffer.to_bytes`` calls
        (src/tensor/runtime/buffer.py:107-112).  This provider's buffers have numpy dtypes (it
        does not offer ``bfloat16_storage``), so storage and value dtypes coincide."""
        result = np.empty(buffer.shape, dtype=buffer.dtype)
        _native.call("tensor_hip_copy_dtoh", result.ctypes.data, buffer.pointer, buffer.nbytes, self.stream)
        return result

    def _download(self, buffer: Buffer) -> np.ndarray:
        return self._download_storage(buffer)

    def _copy(self, destination: Buffer, source: Buffer) -> None:
        if destination.pointer != source.pointer:
            _native.call("tensor_hip_copy_dtod", destination.pointer, source.pointer, source.nbytes, self.stream)

    def _copy_columns(self, destination: Buffer, source: Buffer, offset: int) -> None:
        if (source.pointer < destination.pointer + destination.nbytes
                and destination.pointer < source.pointer + source.nbytes):
            if source.pointer == destination.pointer and source.shape == destination.shape and offset == 0:
                return
            raise ValueError("overlapping column copies are unsupported")
        width = source.dtype.itemsize
        _native.call(
            "tensor_hip_copy_2d",
            destination.pointer + offset * width, destination.shape[1] * width,
            source.pointer, source.shape[1] * width,
            source.shape[1] * width, source.shape[0], self.stream,
        )

    def _dispose_buffer(self, buffer: Buffer) -> None:
        owner = buffer._owner
        if owner is None:
            _native.call("tensor_hip_free", buffer.pointer)
        elif hasattr(owner, "release"):
            owner.release()  # a borrowed DLPack producer goes back to its owner

    # -------------------------------------------------------- executables --
    def load(self, artifact, **options) -> Executable:
        """Load an executable: a built-in GGUF kernel by name (with its options) or manifest
        dict, or a `hip` executable bundle from a path (a hand-built code object; see
        tensor_amd.artifacts), as the reference's ``Device.load(artifact)`` does for its
        bundles (src/tensor/providers/cuda/device.py:359-386)."""
        import os

        from tensor_amd.gguf.kernels import manifest as gguf_manifest

        self._check()
        if isinstance(artifact, os.PathLike) or (isinstance(artifact, str) and os.path.isfile(artifact)):
            if options:
                raise ValueError("options apply only to kernels loaded by name")
            return self._load_bundle(artifact)
        if isinstance(artifact, str):
            manifest = gguf_manifest(artifact, **options)
        elif isinstance(artifact, dict):
            if options:
                raise ValueError("options apply only to kernels loaded by name")
            manifest = artifact
        else:
            raise TypeError("artifact must be a built-in kernel name, a manifest dict or a bundle path")
        if manifest.get("provider") != "hip":
            raise ValueError("artifact requires a different runtime provider")
        check_requirement(manifest["runtime_abi"], self.capabilities)
        if manifest.get("target", self.info["arch"]) != self.info["arch"]:
            raise ValueError(f"artifact target {manifest['target']} does not match device {self.info['arch']}")
        function = _native.kernel(manifest["entrypoint"])
        return Executable(self, manifest, _native.library(), function, None)

    def _load_bundle(self, path) -> Executable:
        from tensor_amd.artifacts import read_artifact
        from tensor_amd.artifacts.hip import IMAGE

        manifest, files = read_artifact(path)  # every member verified before HIP sees a byte
        check_requirement(manifest["runtime_abi"], self.capabilities)
        if manifest["target"] != self.info["arch"]:
            raise ValueError(f"artifact target {manifest['target']} does not match device {self.info['arch']}")
        image = c.create_string_buffer(files[IMAGE], len(files[IMAGE]))
        module, function = c.c_uint64(), c.c_uint64()
        _native.call("tensor_hip_set_device", self.ordinal)
        _native.call("tensor_hip_module_load", c.cast(image, c.c_void_p), len(files[IMAGE]), c.byref(module))
        try:
            _native.call("tensor_hip_module_function", module.value, manifest["entrypoint"].encode(), c.byref(function))
        except BaseException:
            _native.call("tensor_hip_module_unload", module.value)
            raise
        return Executable(self, manifest, module.value, function.value, image)

    def _unload_executable(self, executable) -> None:
        if executable.manifest.get("kind") == "hsaco":
            _native.call("tensor_hip_module_unload", executable.module)
        # built-in entry points live for the life of the process-wide library

    def _launch(self, executable, call) -> None:
        self._make_current()
        if self._capture_log is not None:
            self._capture_log.extend(call.storage)
        error = ErrorDescriptor()
        if executable.manifest.get("kind") == "hsaco":
            module_launch = _native.library().tensor_hip_module_launch_v1

            def submit():
                return module_launch(executable.function, c.byref(call.descriptor), c.byref(error))
        else:
            entry = executable.function

            def submit():
                return entry(c.byref(call.descriptor), c.byref(error))
        status = submit()
        if status == 3 and _NOT_CURRENT in error.message:
            self._check()  # another caller moved this thread's device; the call was not enqueued
            status = submit()
        if status:
            raise HipError(executable.manifest["entrypoint"], status, error.message.decode(errors="replace"))

    # -------------------------------------------------------------- events --
    def record_event(self, *, timing: bool = False) -> Event:
        self._check()
        handle = c.c_uint64()
        _native.call("tensor_hip_event_create", c.byref(handle), int(timing))
        try:
            _native.call("tensor_hip_event_record", handle.value, self.stream)
        except BaseException:
            _native.call("tensor_hip_event_destroy", handle.value)
            raise
        return Event(self, handle.value)

    def wait(self, event: Event) -> None:
        self._check()
        event._check(self)
        _native.call("tensor_hip_stream_wait_event", self.stream, event.handle)

    def elapsed_ms(self, start: Event, stop: Event) -> float:
        """Milliseconds between two timing events recorded on this stream."""
        start._check(self)
        stop._check(self)
        value = c.c_float()
        _native.call("tensor_hip_event_elapsed", c.byref(value), start.handle, stop.handle)
        return value.value

    def _synchronize_event(self, event: Event) -> None:
        _native.call("tensor_hip_event_synchronize", event.handle)

    def _dispose_event(self, event: Event) -> None:
        _native.call("tensor_hip_event_destroy", event.handle)

    # -------------------------------------------------------------- graphs --
    def gemm_workspace(self, encoding, m: int, k: int, rows) -> int:
        """Bytes of workspace ``gguf_gemm_group`` uses for this shape (``rows`` = each matrix's
        N); 0 when it does not split K.  A smaller workspace is accepted and limits the split."""
        from tensor_amd.gguf.quant import ggml_type

        rows = [int(n) for n in rows]
        result = c.c_uint64()
        _native.call("tensor_gguf_gemm_workspace_v1", ggml_type(encoding), int(m), int(k),
                     (c.c_int64 * len(rows))(*rows), len(rows), c.byref(result))
        return result.value

    def gemv_plan(self, encoding, m: int, k: int, n: int) -> dict | None:
        """The multi-row plan ``gguf_gemv`` takes for a Q4_K call with 2 <= m <= 8 (None where
        the call takes another path): the kernel (``GEMV_KERNELS``) and its two launch fields,
        which ``gguf_gemv_variant`` accepts as its ``kernel``, ``a`` and ``b`` scalars."""
        from tensor_amd.gguf.quant import ggml_type

        kernel, a, b = c.c_int32(), c.c_int32(), c.c_int32()
        _native.call("tensor_gguf_gemv_plan_v1", ggml_type(encoding), int(m), int(k), int(n), c.byref(kernel),
                     c.byref(a), c.byref(b))
        if kernel.value < 0:
            return None
        return {"kernel": kernel.value, "name": GEMV_KERNELS[kernel.value], "a": a.value, "b": b.value}

    def gemm_plan(self, encoding, m: int, k: int, rows, workspace_bytes: int | None = None) -> dict:
        """The plan ``gguf_gemm_group`` takes for this shape (``workspace_bytes`` of workspace,
        by default as much as it asks for): tile index, its geometry, the K split, and whether
        the pipelined kernel runs (otherwise each matrix takes the small-M kernel)."""
        from tensor_amd.gguf.quant import ggml_type

        rows = [int(n) for n in rows]
        if workspace_bytes is None:
            workspace_bytes = self.gemm_workspace(encoding, m, k, rows)
        tile, splits, pipelined = c.c_int32(), c.c_int32(), c.c_int32()
        _native.call("tensor_gguf_gemm_plan_v1", ggml_type(encoding), int(m), int(k), (c.c_int64 * len(rows))(*rows),
                     len(rows), int(workspace_bytes), c.byref(tile), c.byref(splits), c.byref(pipelined))
        return dict(gemm_tiles()[tile.value], tile=tile.value, splits=splits.value, pipelined=bool(pipelined.value))

    def graph(self, callback, *, resources=()):
        """Capture the launches ``callback()`` enqueues into a replayable graph.  The buffers of
        every call launched during the capture, and ``resources``, are checked before each
        replay."""
        from tensor_amd.providers.hip_graph import HipGraph

        return HipGraph(self, callback, resources=resources)

    # ------------------------------------------------------------ teardown --
    def _cleanup(self) -> None:
        errors = []

        def attempt(function, *arguments):
            try:
                function(*arguments)
            except HipError as exc:
                errors.append(exc)

        if self._open:
            attempt(_native.call, "tensor_hip_set_device", self.ordinal)
            attempt(_native.call, "tensor_hip_stream_synchronize", self.stream)
            for handle in self._consumers:
                attempt(_native.call, "tensor_hip_stream_synchronize", handle)
        for graph in list(self._graphs):
            attempt(graph._dispose)
        for event in list(self._events):
            attempt(event.release)
        for buffer in list(self._buffers):
            attempt(buffer._dispose)
        for executable in list(getattr(self, "_executables", {}).values()):
            attempt(executable._dispose)
        if self._open and self.owns_stream and self.stream:
            attempt(_native.call, "tensor_hip_stream_destroy", self.stream)
        self._open = False
        self._buffers.clear()
        self._consumers.clear()
        self._graphs.clear()
        self.stream = 0
        if errors:
            raise errors[0]

    def __exit__(self, exc_type, exc, tb) -> None:
        try:
            self._cleanup()
        except HipError:
            if exc_type is None:
                raise

    @contextlib.contextmanager
    def session(self):
        with self:
            yield self
