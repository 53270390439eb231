"""PyTorch-ROCm interop on the GPU: tensor_amd.torch kernels on torch tensors and
kDLROCM DLPack exchange both ways.

The checks run in a child process (tests/torch_interop.py) that imports torch
before the library is loaded, so both use torch's HIP runtime; this process
may already have bound libtensor_hip.so to the system runtime.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.timeout(480)
@pytest.mark.parametrize("native", ["1", "0"], ids=["native-executor", "python-launch"])
def test_torch_interop_in_a_torch_first_process(native):
    print(f"[case] torch-interop child TENSOR_AMD_TORCH_NATIVE={native}", flush=True)
    result = subprocess.run([sys.executable, "-u", str(ROOT / "tests" / "torch_interop.py")], cwd=ROOT,
                            capture_output=True, text=True, timeout=420,
                            env=dict(os.environ, PYTHONPATH=str(ROOT), TENSOR_AMD_TORCH_NATIVE=native))
    print(result.stdout[-4000:], result.stderr[-4000:], flush=True)
    assert result.returncode == 0, result.stderr[-2000:]
    assert "[torch-interop] ok" in result.stdout
