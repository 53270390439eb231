"""Build libtensor_hip.so in-tree with hipcc for gfx950.

``python -m tensor_amd.build`` (or ``__graft_entry__.build()``) compiles every
``csrc/*.hip`` translation unit in parallel and links the shared library next
to this file, where the provider loads it; it also compiles every hand-written
kernel under ``kernels/`` to an unbundled gfx950 code object and packs it into a
`hip` executable bundle (``kernels/<name>.tbin``).  There is no JIT path: a
missing library or bundle is an error at load time, never a fallback.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libtensor_hip.so"
ARCH = os.environ.get("TENSOR_HIP_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (unreliable on this pool).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

# The library's kernels take their leading scalar arguments preloaded into SGPRs by the
# dispatcher (gfx950 kernel-argument preloading), so a wave's first loads do not wait on
# scalar loads of the argument block; on firmware without the feature the compiler's
# entry sequence loads the same registers itself.
LIBRARY_FLAGS = [*DEVICE_FLAGS, "-mllvm", "-amdgpu-kernarg-preload-count=16"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build tensor_amd")


def _compile(source: Path, verbose: bool) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [hipcc(), *LIBRARY_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")
    if verbose and result.stderr.strip():
        print(result.stderr, file=sys.stderr)
    return obj


KERNELS = PACKAGE / "kernels"


def _compiler_version() -> str:
    result = subprocess.run([hipcc(), "--version"], capture_output=True, text=True)
    lines = [line.strip() for line in result.stdout.splitlines() if line.strip()]
    return "; ".join(lines[:2]) if lines else "unknown"


def build_bundles(verbose: bool = False) -> list:
    """Compile kernels/<name>.hip to a code object and pack kernels/<name>.tbin."""
    from tensor_amd.artifacts import write_artifact
    from tensor_amd.kernels import BUNDLES

    built = []
    version = _compiler_version()
    for name, spec in BUNDLES.items():
        source = KERNELS / f"{name}.hip"
        code_object = KERNELS / f"{name}.hsaco"
        cmd = [hipcc(), "--genco", "--no-gpu-bundle-output", *DEVICE_FLAGS, str(source), "-o", str(code_object)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode:
            raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")
        if verbose and result.stderr.strip():
            print(result.stderr, file=sys.stderr)
        bundle = KERNELS / f"{name}.tbin"
        write_artifact(bundle, code_object.read_bytes(), name=name, target=ARCH,
                       compiler={"name": "hipcc", "version": version}, source=source.read_bytes(), **spec)
        built.append(bundle)
    return built


EXECUTOR = PACKAGE / "torch" / "executor.cpp"


def executor_module() -> str:
    """Module name of the native executor for the installed torch (its major/minor)."""
    import torch

    major, minor = torch.__version__.split("+")[0].split(".")[:2]
    return f"_executor_{major}_{minor}"


def build_executor(verbose: bool = False) -> Path | None:
    """Compile tensor_amd.torch's native executor against the installed PyTorch-ROCm
    (host C++ only, g++; it calls the provider's C ABI).  Skipped without torch."""
    try:
        import torch
        from torch.utils import cpp_extension
    except ImportError:
        return None
    if torch.version.hip is None:
        return None
    import sysconfig

    name = executor_module()
    target = EXECUTOR.parent / f"{name}.so"
    tmp = target.with_suffix(".so.tmp")
    torch_lib = Path(torch.__file__).parent / "lib"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-DTENSOR_EXECUTOR_MODULE={name}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *(f"-I{path}" for path in cpp_extension.include_paths()),
        f"-I{sysconfig.get_paths()['include']}", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
        str(EXECUTOR), f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{torch_lib}", "-o", str(tmp),
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"executor build failed:\n{result.stdout}\n{result.stderr}")
    if verbose and result.stderr.strip():
        print(result.stderr, file=sys.stderr)
    os.replace(tmp, target)
    return target


def source_hash() -> str:
    """SHA-256 over the compiler flags (include paths aside) and every file the library is
    compiled from (csrc/ and include/, by relative path and content).  build() embeds it in
    the library and the loader refuses a library whose embedded hash differs from the sources
    beside it, so a stale binary is never tested or benchmarked silently."""
    import hashlib

    digest = hashlib.sha256()
    digest.update(" ".join(f for f in LIBRARY_FLAGS if not f.startswith("-I")).encode() + b"\0")
    files = sorted(p for d in (CSRC, ROOT / "include") for p in d.rglob("*") if p.is_file())
    for path in files:
        digest.update(str(path.relative_to(ROOT)).encode() + b"\0")
        digest.update(path.read_bytes())
        digest.update(b"\0")
    return digest.hexdigest()


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    identity = source_hash()
    stamp = BUILD / "source_hash.c"
    stamp.write_text(f'const char* tensor_hip_source_hash(void) {{ return "{identity}"; }}\n')
    stamp_obj = BUILD / "source_hash.o"
    result = subprocess.run([os.environ.get("CC", "gcc"), "-O2", "-fPIC", "-c", str(stamp), "-o", str(stamp_obj)],
                            capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"source hash stamp failed:\n{result.stderr}")
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources)) + [stamp_obj]
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    build_bundles(verbose)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
