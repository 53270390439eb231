"""Provider-neutral runtime: buffers, executables, bound calls, events, sessions."""

from tensor_amd.runtime.buffer import Buffer, BufferView
from tensor_amd.runtime.errors import TensorRuntimeError
from tensor_amd.runtime.event import Event
from tensor_amd.runtime.executable import Executable
from tensor_amd.runtime.session import Session
from tensor_amd.runtime.timing import bench

__all__ = ["Buffer", "BufferView", "Executable", "Event", "Session", "TensorRuntimeError", "bench"]
