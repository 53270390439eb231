"""Shared fixtures.  ``gpu`` tests need an MI355X and the built library; the CPU
suite (``-m "not gpu"``) covers the oracle, host logic and ABI validation."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libtensor_hip.so")


@pytest.fixture(scope="session")
def c_oracle():
    from oracle import gguf_ref

    if not gguf_ref.LIBRARY.exists():
        gguf_ref.build()
    return gguf_ref.c_oracle()


@pytest.fixture(scope="session")
def hip_device():
    """One HIP session for the whole GPU suite (a single process on the card)."""
    import tensor_amd as tx

    device = tx.Device(0, provider="hip")
    with device:
        print(f"[hip] {device.info['name']} {device.info['arch_features']} "
              f"CUs={device.info['compute_units']}", flush=True)
        yield device
