"""HIP provider sessions and current-stream lookup for PyTorch-ROCm callers.

Follows packages/tensor-torch/src/tensor_torch/runtime/session.py:10-33 and
runtime/streams.py:8-24: one provider session per device, retained until
``close()``; launch streams are PyTorch's current stream, chosen per call.

One process, one HIP runtime: a PyTorch-ROCm wheel ships its own libamdhip64
under the system library's soname, so when torch is imported before
libtensor_hip.so is first loaded (importing this package does that), both use
torch's runtime.  Loaded the other way round, the process holds two HIP
runtimes whose streams and pointers do not mix; sessions are then refused.
"""

from __future__ import annotations

import atexit
import threading

import torch

_sessions: dict = {}
_streams: dict = {}
_lock = threading.RLock()


def hip_runtimes() -> set:
    """Paths of the HIP runtime libraries mapped into this process."""
    paths = set()
    with open("/proc/self/maps") as maps:
        for line in maps:
            fields = line.split()
            if len(fields) >= 6 and "libamdhip64" in fields[-1]:
                paths.add(fields[-1])
    return paths


def _check_single_runtime() -> None:
    paths = hip_runtimes()
    if len(paths) > 1:
        raise RuntimeError(f"two HIP runtimes are loaded ({', '.join(sorted(paths))}): import torch (or "
                           "tensor_amd.torch) before the first tensor_amd device is opened")


def session(ordinal: int):
    """This process's HIP provider session for one device, opened on first use.  Its own
    stream is PyTorch's current stream at that moment; launches name theirs per call."""
    from tensor_amd.providers.hip import Device

    with _lock:
        device = _sessions.get(ordinal)
        if device is None or not device._open:
            _check_single_runtime()
            device = Device(ordinal, stream=torch.cuda.current_stream(ordinal).cuda_stream)
            device.__enter__()
            _sessions[ordinal] = device
        return device


def current_stream(ordinal: int):
    """PyTorch's current stream on ``ordinal`` (a torch.cuda.Stream), cached by handle."""
    getter = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if getter is None:
        return torch.cuda.current_stream(ordinal)
    key = (ordinal, getter(ordinal))
    stream = _streams.get(key)
    if stream is None:
        stream = _streams[key] = torch.cuda.current_stream(ordinal)
    return stream


def close() -> None:
    """Wait for the devices, then close every session this package opened.  PyTorch's
    allocations are never released here: torch owns them."""
    with _lock:
        for device in _sessions.values():
            if device._open:
                with torch.cuda.device(device.ordinal):
                    torch.cuda.synchronize()
                device.__exit__(None, None, None)
        _sessions.clear()
        _streams.clear()


atexit.register(close)
