"""ctypes binding of libtensor_hip.so (declarations: include/tensor_hip.h).

The library is built in-tree (``python -m tensor_amd.build``).  A missing or
unloadable library raises ``NativeLibraryError``; there is no fallback path.
"""

from __future__ import annotations

import ctypes as c
import threading
from pathlib import Path

from tensor_amd.runtime.abi import CallDescriptor, ErrorDescriptor
from tensor_amd.runtime.errors import TensorRuntimeError

LIBRARY = Path(__file__).resolve().parent / "libtensor_hip.so"

# Kernel entry points (TensorKernelV1 shape).
KERNELS = (
    "tensor_gguf_packed_v1",
    "tensor_gguf_gemm_group_v1",
    "tensor_gguf_gemm_group_noalloc_v1",
    "tensor_gguf_gemm_group_plan_v1",
    "tensor_gguf_gemv_v1",
    "tensor_gguf_gemm_v1",
    "tensor_gguf_linear_v1",
    "tensor_gguf_gemv_group_v1",
    "tensor_gguf_gemv_swiglu_v1",
    "tensor_gguf_gemv_variant_v1",
    "tensor_gguf_gemv_q8_1_v1",
    "tensor_gguf_dequant_v1",
)

_u64, _i32, _f32p = c.c_uint64, c.c_int32, c.POINTER(c.c_float)
_err = c.POINTER(ErrorDescriptor)


class TensorHipDeviceInfo(c.Structure):
    _fields_ = [
        ("name", c.c_char * 256),
        ("arch", c.c_char * 64),
        ("total_memory", c.c_uint64),
        ("l2_cache_bytes", c.c_uint64),
        ("compute_units", c.c_int32),
        ("clock_khz", c.c_int32),
        ("memory_clock_khz", c.c_int32),
        ("memory_bus_width", c.c_int32),
        ("max_threads_per_block", c.c_int32),
        ("max_shared_memory_per_block", c.c_int32),
        ("warp_size", c.c_int32),
        ("max_grid", c.c_int32 * 3),
        ("max_block", c.c_int32 * 3),
    ]


# Runtime services: name -> argument types (every one ends with TensorErrorV1*).
SERVICES = {
    "tensor_hip_device_count": [c.POINTER(_i32)],
    "tensor_hip_device_info": [_i32, c.POINTER(TensorHipDeviceInfo)],
    "tensor_hip_set_device": [_i32],
    "tensor_hip_device_synchronize": [],
    "tensor_hip_malloc": [_u64, c.POINTER(_u64)],
    "tensor_hip_free": [_u64],
    "tensor_hip_pointer_device": [_u64, c.POINTER(_i32), c.POINTER(_i32)],
    "tensor_hip_copy_htod": [_u64, c.c_void_p, _u64, _u64],
    "tensor_hip_copy_dtoh": [c.c_void_p, _u64, _u64, _u64],
    "tensor_hip_copy_dtod": [_u64, _u64, _u64, _u64],
    "tensor_hip_copy_2d": [_u64, _u64, _u64, _u64, _u64, _u64, _u64],
    "tensor_hip_fill_u8": [_u64, c.c_uint8, _u64, _u64],
    "tensor_hip_stream_create": [c.POINTER(_u64)],
    "tensor_hip_stream_destroy": [_u64],
    "tensor_hip_stream_synchronize": [_u64],
    "tensor_hip_stream_wait_event": [_u64, _u64],
    "tensor_hip_event_create": [c.POINTER(_u64), _i32],
    "tensor_hip_event_destroy": [_u64],
    "tensor_hip_event_record": [_u64, _u64],
    "tensor_hip_event_synchronize": [_u64],
    "tensor_hip_event_query": [_u64, c.POINTER(_i32)],
    "tensor_hip_event_elapsed": [_f32p, _u64, _u64],
    "tensor_hip_capture_begin": [_u64],
    "tensor_hip_capture_end": [_u64, c.POINTER(_u64)],
    "tensor_hip_graph_launch": [_u64, _u64],
    "tensor_hip_graph_destroy": [_u64],
    "tensor_hip_module_load": [c.c_void_p, _u64, c.POINTER(_u64)],
    "tensor_hip_module_function": [_u64, c.c_char_p, c.POINTER(_u64)],
    "tensor_hip_module_unload": [_u64],
    "tensor_gguf_gemm_workspace_v1": [c.c_uint32, c.c_int64, c.c_int64, c.POINTER(c.c_int64), c.c_uint32,
                                      c.POINTER(_u64)],
    "tensor_gguf_gemm_plan_v1": [c.c_uint32, c.c_int64, c.c_int64, c.POINTER(c.c_int64), c.c_uint32, _u64,
                                 c.POINTER(_i32), c.POINTER(_i32), c.POINTER(_i32)],
    "tensor_gguf_gemm_tile_v1": [_i32, c.POINTER(_i32), c.POINTER(_i32), c.POINTER(_i32)],
    "tensor_gguf_gemv_plan_v1": [c.c_uint32, c.c_int64, c.c_int64, c.c_int64, c.POINTER(_i32), c.POINTER(_i32),
                                 c.POINTER(_i32)],
}


class NativeLibraryError(TensorRuntimeError):
    pass


class HipError(TensorRuntimeError):
    """A failed library call: ``code`` is the TENSOR_ERROR_* status."""

    def __init__(self, function: str, code: int, message: str):
        super().__init__(f"{function}: {message} ({code})")
        self.function, self.code, self.message = function, code, message


_lock = threading.Lock()
_library = None


def library(path: Path | None = None) -> c.CDLL:
    """Load (once) and type the native library."""
    global _library
    with _lock:
        if _library is not None and path is None:
            return _library
        target = Path(path) if path is not None else LIBRARY
        if not target.exists():
            raise NativeLibraryError(
                f"{target} is not built; run `python -m tensor_amd.build` (hipcc, gfx950)"
            )
        try:
            lib = c.CDLL(str(target))
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {target}: {exc}") from exc
        for name in KERNELS:
            function = getattr(lib, name)
            function.argtypes = [c.POINTER(CallDescriptor), _err]
            function.restype = c.c_int32
        for name, argtypes in SERVICES.items():
            function = getattr(lib, name)
            function.argtypes = [*argtypes, _err]
            function.restype = c.c_int32
        lib.tensor_hip_module_launch_v1.argtypes = [_u64, c.POINTER(CallDescriptor), _err]
        lib.tensor_hip_module_launch_v1.restype = c.c_int32
        lib.tensor_hip_version.argtypes = []
        lib.tensor_hip_version.restype = c.c_char_p
        lib.tensor_hip_source_hash.argtypes = []
        lib.tensor_hip_source_hash.restype = c.c_char_p
        if path is None:
            _check_fresh(lib, target)
            _library = lib
        return lib


def _check_fresh(lib: c.CDLL, target: Path) -> None:
    """Refuse a library built from other sources than the csrc/ and include/ beside it."""
    from tensor_amd import build

    if not build.CSRC.is_dir():
        return  # an installed library without its sources: nothing to compare
    embedded = lib.tensor_hip_source_hash().decode()
    current = build.source_hash()
    if embedded != current:
        raise NativeLibraryError(
            f"{target} was built from other sources ({embedded[:12]}) than tensor_amd/csrc and include "
            f"({current[:12]}); rebuild with `python -m tensor_amd.build`"
        )


def call(name: str, *arguments) -> None:
    """Invoke a runtime service and raise HipError on failure."""
    error = ErrorDescriptor()
    status = getattr(library(), name)(*arguments, c.byref(error))
    if status:
        raise HipError(name, status, error.message.decode(errors="replace"))


def kernel(name: str):
    if name not in KERNELS:
        raise NativeLibraryError(f"unknown kernel entry point {name!r}")
    return getattr(library(), name)
