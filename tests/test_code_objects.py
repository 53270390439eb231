"""Every gfx950 kernel in libtensor_hip.so fits the resources the part and HIP allow, read from
the code objects' own AMDGPU metadata (CPU only: the library's .hip_fatbin section is parsed,
nothing is loaded on a GPU).

A code object the runtime cannot load fails at the process's first launch from the library,
whichever kernel that launch names, so the limits are checked for every kernel at build time:
LDS per workgroup (160 KiB on gfx950), the unified VGPR + AGPR file (512 per lane), SGPRs, the
kernel-argument segment, workgroup size, wave size, no dynamic call stack, and scratch only for
the instantiations listed here with their reason.
"""

from __future__ import annotations

import re

import pytest

from tensor_amd import _native
from tensor_amd.artifacts.hip import code_object_metadata, offload_code_objects

LDS_BYTES = 160 * 1024
VGPR_FILE = 512
SGPRS = 106           # addressable SGPRs, VCC included
KERNARG_BYTES = 4096  # HIP's limit on a kernel's explicit arguments
# gemv_q4k_mt with two 16-row tiles per wave and three super-blocks (K of 8448 .. 12288, x in
# LDS, N >= 8192 and no sector-kernel shape) keeps 4 VGPRs of its second tile's codes in
# scratch; every other kernel runs without a private segment.
SCRATCH_ALLOWED = re.compile(r"gemv_q4k_mtILi\dELi2ELi3E")


@pytest.fixture(scope="module")
def kernels():
    path = _native.LIBRARY
    if not path.exists():
        pytest.skip("libtensor_hip.so is not built")
    objects = offload_code_objects(path.read_bytes())
    assert objects, "no gfx950 code object in the library"
    records = []
    for image in objects:
        metadata = code_object_metadata(image)
        assert metadata["amdhsa.target"].startswith("amdgcn-amd-amdhsa--gfx950"), metadata["amdhsa.target"]
        records += metadata["amdhsa.kernels"]
    return records


def test_library_carries_the_hot_path_kernels(kernels):
    names = {k[".name"] for k in kernels}
    for stem in ("gemv_q4k_m1", "gemv_q4k_sec", "gemv_q6k_lds", "gemv_q32_m1", "gemm_pipe", "gemm_reduce",
                 "gemm_skinny", "dequant_kernel"):
        assert any(stem in name for name in names), stem


def test_every_kernel_fits_gfx950(kernels):
    bad = []
    for k in kernels:
        name = k[".name"]
        problems = []
        if k[".group_segment_fixed_size"] > LDS_BYTES:
            problems.append(f"LDS {k['.group_segment_fixed_size']}")
        if k[".vgpr_count"] + k.get(".agpr_count", 0) > VGPR_FILE:
            problems.append(f"VGPR {k['.vgpr_count']} + AGPR {k.get('.agpr_count', 0)}")
        if k[".sgpr_count"] > SGPRS:
            problems.append(f"SGPR {k['.sgpr_count']}")
        if k[".kernarg_segment_size"] > KERNARG_BYTES:
            problems.append(f"kernarg {k['.kernarg_segment_size']}")
        if k[".max_flat_workgroup_size"] > 1024 or k[".wavefront_size"] != 64:
            problems.append(f"workgroup {k['.max_flat_workgroup_size']} wave {k['.wavefront_size']}")
        if k.get(".uses_dynamic_stack"):
            problems.append("dynamic stack")
        if k[".private_segment_fixed_size"] and not SCRATCH_ALLOWED.search(name):
            problems.append(f"scratch {k['.private_segment_fixed_size']} B")
        if problems:
            bad.append((name, problems))
    assert not bad, bad[:10]
