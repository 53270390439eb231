"""Runtime contract errors (reference: src/tensor/runtime/errors.py)."""

from __future__ import annotations


class TensorRuntimeError(RuntimeError):
    pass
