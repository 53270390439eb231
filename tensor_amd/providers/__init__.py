"""Runtime provider selection (reference: src/tensor/providers/__init__.py:10-36).

This package provides the ROCm provider ``"hip"``; the factory keeps the
reference's signature so caller code reads ``Device(provider="hip")``.
"""

from importlib import import_module

PROVIDERS = {
    "hip": "tensor_amd.providers.hip",
}


def Device(ordinal=0, *, provider="hip", stream=None, require_capabilities=(), max_buffer_size=None):
    if provider not in PROVIDERS:
        raise ValueError(f"unknown runtime provider {provider!r}; choose {', '.join(PROVIDERS)}")
    implementation = import_module(PROVIDERS[provider]).Device
    missing = set(require_capabilities) - implementation.capabilities
    if missing:
        raise ValueError(f"provider {provider} lacks capabilities: {sorted(missing)}")
    if max_buffer_size is not None:
        raise ValueError("max_buffer_size is only supported by the WebGPU provider")
    return implementation(ordinal, stream=stream)
