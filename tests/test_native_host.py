"""A compiled C++ host drives libtensor_hip.so through the public headers alone.

Mirrors the reference's native-host test (tests/runtime/test_runtime_abi.py:187-194,
host src/tensor/native/host.cpp:51-131): g++ builds tensor_amd/native/host.cpp
against include/ only, the host dlopens the library and calls its entry points
with TensorCallV1 descriptors.  The malformed calls fail before any HIP call, so
``check`` runs on a machine without a GPU; ``gpu`` adds real calls whose
products are exact.
"""

from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIBRARY = ROOT / "tensor_amd" / "libtensor_hip.so"


@pytest.fixture(scope="module")
def host(tmp_path_factory):
    binary = tmp_path_factory.mktemp("native") / "host"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-I", str(ROOT / "include"),
                    str(ROOT / "tensor_amd" / "native" / "host.cpp"), "-ldl", "-o", str(binary)],
                   check=True, capture_output=True)
    return binary


def run(host, mode):
    result = subprocess.run([str(host), mode, str(LIBRARY)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stderr
    return json.loads(result.stdout)


def test_native_host_refuses_malformed_calls_before_any_hip_call(host):
    report = run(host, "check")
    assert report["status"] == "passed" and report["negative_checks"] == 14


@pytest.mark.gpu
def test_native_host_runs_the_packed_form_on_the_gpu(host):
    print("[case] native host gpu", flush=True)
    report = run(host, "gpu")
    assert report == {"status": "passed", "mode": "gpu", "abi": 1, "negative_checks": 14, "exact_calls": 2}
