"""PyTorch-ROCm binding of the HIP provider's executables.

The counterpart of the reference's tensor-torch package
(packages/tensor-torch/src/tensor_torch/__init__.py, loading.py:8-34):
``load`` returns a ``Kernel`` registered as a functional custom operator whose
call allocates the declared outputs with torch, binds the call ABI once per
shape through kDLROCM DLPack and submits on ``torch.cuda.current_stream()``.
The reference's FX compile backend and module references are not part of this
binding.

Import torch (or this package) before the first tensor_amd device is opened:
the library then shares torch's HIP runtime.
"""

from __future__ import annotations

import torch  # noqa: F401  (first: the process's HIP runtime is torch's)

from tensor_amd.torch.kernel import Kernel
from tensor_amd.torch.session import close, hip_runtimes

__all__ = ["Kernel", "close", "hip_runtimes", "load"]


def load(artifact, **options) -> Kernel:
    """A registered Kernel for a built-in GGUF kernel name (with its options), a manifest
    dict or a ``hip`` bundle path.  Module references (``module::export``) need the
    reference's module registry and are refused."""
    if isinstance(artifact, str) and "::" in artifact:
        raise ValueError("module references are not supported; load a kernel name or a hip bundle")
    kernel = Kernel(artifact, **options)
    kernel.register()
    return kernel
