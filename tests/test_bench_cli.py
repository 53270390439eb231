"""bench.py's command line on the CPU: it compiles and refuses more than one GPU before it
touches a device (the driver runs it at round end; a syntax error would lose the bench)."""

from __future__ import annotations

import py_compile
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_compiles():
    py_compile.compile(str(ROOT / "bench.py"), doraise=True)


def test_bench_refuses_several_gpus_without_a_device():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                            capture_output=True, text=True, timeout=120)
    assert result.returncode == 2
    assert "one GPU" in result.stderr
