"""A hand-built code object loaded from a `hip` executable bundle (Device.load(path)) and
launched through the module entry point, as the reference's provider loads its bundles
(src/tensor/providers/cuda/device.py:359-386) and launches them (:211-229): the shipped
SwiGLU kernel (tensor_amd/kernels/swiglu.hip) against a float64 NumPy reference, bound
and replayed from a captured graph, released and unloaded."""

from __future__ import annotations

import numpy as np
import pytest

from tensor_amd.kernels import bundle_path

pytestmark = pytest.mark.gpu


def reference(gate, up):
    g = gate.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * up.astype(np.float64)


def close_enough(got, want):
    # one fp16 rounding of a value computed in fp32: |error| <= 2^-11 |want| plus fp32 slack
    return np.all(np.abs(got.astype(np.float64) - want) <= 1e-3 * np.abs(want) + 1e-6)


@pytest.mark.parametrize("m,n", [(1, 12288), (3, 1001), (1, 7)])
def test_swiglu_bundle_matches_numpy(hip_device, m, n):
    print("[case] swiglu bundle", m, n, flush=True)
    kernel = hip_device.load(str(bundle_path("swiglu")))
    rng = np.random.default_rng(m * n)
    gate = (rng.standard_normal((m, n)) * 3).astype(np.float16)
    up = rng.standard_normal((m, n)).astype(np.float16)
    gb, ub = hip_device.from_numpy(gate), hip_device.from_numpy(up)
    out = kernel(gb, ub)  # the declared output is allocated; M and N bind from the shapes
    got = out.to_numpy()
    assert got.shape == (m, n) and got.dtype == np.float16
    assert close_enough(got, reference(gate, up))
    for b in (gb, ub, out):
        b.release()
    kernel.release()


def test_swiglu_bundle_graph_replay_sees_new_inputs(hip_device):
    kernel = hip_device.load(bundle_path("swiglu"))  # a PathLike works as well as a str
    m, n = 2, 4096
    rng = np.random.default_rng(7)
    gate = hip_device.from_numpy(rng.standard_normal((m, n)).astype(np.float16))
    up = hip_device.from_numpy(rng.standard_normal((m, n)).astype(np.float16))
    out = hip_device.empty((m, n), "float16")
    call = kernel.bind(gate, up, out)
    graph = hip_device.graph(call.launch)
    try:
        for seed in (11, 12, 13):
            g = np.random.default_rng(seed).standard_normal((m, n)).astype(np.float16)
            u = np.random.default_rng(seed + 100).standard_normal((m, n)).astype(np.float16)
            staged = [hip_device.from_numpy(g), hip_device.from_numpy(u)]
            gate.copy_from(staged[0])
            up.copy_from(staged[1])
            hip_device.fill_bytes(out, 0xFF)
            graph.replay()
            assert close_enough(out.to_numpy(), reference(g, u)), seed
            for b in staged:
                b.release()
    finally:
        graph.close()
    for b in (gate, up, out):
        b.release()
    kernel.release()


def test_bundle_shape_mismatch_is_refused_before_launch(hip_device):
    kernel = hip_device.load(str(bundle_path("swiglu")))
    gate = hip_device.from_numpy(np.zeros((2, 64), np.float16))
    up = hip_device.from_numpy(np.zeros((2, 32), np.float16))
    with pytest.raises(Exception, match="N|shape"):
        kernel(gate, up)
    for b in (gate, up):
        b.release()
    kernel.release()
