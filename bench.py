"""Benchmark of the GGUF quantized-linear hot path on one MI355X.

Headline ("C2"): Q4_K decode GEMV at Qwen3-8B MLP
shapes, M = 1.  One *step* is one decode MLP's linears through the C ABI: gate
[12288 x 4096] and up [12288 x 4096] as one grouped launch (they share x), then
down [4096 x 12288].  ``value`` is the algorithmic bytes of all K steps
(packed weights + fp16 x + fp16 out) divided by the timed region.

Timing protocol (after benchmarks/kernels/showcase/benchmark.py:66-94 and
:1007-1013): every launch is bound once (allocation-free BoundCall), a case's
launches are captured into one HIP graph, the graph is replayed REPLAYS (>= 11)
times with HIP events recorded on the launch stream around each replay, and
the case reports the median, min, max and every sample.  The detail cases run
in a seeded shuffled order, kept in the output.  Weights rotate through
distinct copies (>= 3 x 256 MiB per rotation) so no launch finds its weights in
the 256 MiB MALL, except the showcase cases, which keep the reference's
hot-cache protocol (one weight copy, N = K = 1024).  Before the timed replays
every sequence is replayed, untimed, for WARM_SECONDS: an MI355X that has idled
through the host-side set-up of a case starts in deep sleep and needs ~30 ms of
sustained load to reach its steady clocks (measured on the LM head: 123 us per
launch over the first 100 launches, 93 us from the fourth hundred on).

Also reported:

* ``roofline`` for the dominant kernel (the grouped gate + up GEMV, 2 x
  12288 x 4096): ``avg_us``, ``achieved``, ``frac`` and HBM ``traffic`` from
  the committed rocprofv3 summary (profiles/gemv_q4k_m1_qwen3_mlp.md), and this
  run's own HIP-event timings under ``live``: per launch of 200 eager launches
  and of the same launches captured in a graph;
* ``cpu_baseline``: the C restatement in oracle/, invoked through its
  TensorKernelV1 entries exactly as the reference CPU provider invokes images,
  on the headline step and on every other configuration (``per_config``:
  decode numerics for the GEMV configs, prefill numerics for the GEMM ones);
* ``details`` for the other BASELINE configurations (C1's shape, C2 M = 4/8,
  C3 LM head, C4 prefill GEMM, C5 decoder-layer chain at M = 1 and M = 256),
  the showcase's packed call at its own shapes, and the resident-dequantized
  torch.mm lower bound (benchmark.py:478-488) measured in a torch-first child.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FP16_PEAK_TFLOPS = 2516.6   # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20
ROTATION_BYTES = 3 * MALL_BYTES
REPLAYS = 11                # timed replays per case (median, min, max and samples reported)
METRIC = "Q4_K/Q6_K decode GEMV GB/s (% HBM peak); prefill dequant-GEMM TFLOP/s"
GEOMETRY = {"q4_0": (32, 18), "q8_0": (32, 34), "q4_k": (256, 144), "q6_k": (256, 210), "q4_1": (32, 20),
            "q5_0": (32, 22), "q5_1": (32, 24), "q2_k": (256, 84), "q3_k": (256, 110), "q5_k": (256, 176)}
# The reference's published showcase figures (NVIDIA L4, hot L2, research/studies/cuda-showcase/
# evidence/l4-20261024/REPORT.md:19-24): context for the showcase cases, not a same-node target.
L4_SHOWCASE_US = {("q4_0", 1): 2.355, ("q4_0", 32): 8.924, ("q4_k", 1): 2.729, ("q4_k", 32): 13.829,
                  ("q6_k", 1): 3.261, ("q6_k", 32): 13.332}


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def weight_bytes(encoding, n, k):
    qk, block = GEOMETRY[encoding]
    return n * (k // qk) * block


def gemv_bytes(encoding, m, n, k, out_itemsize, x_itemsize=2):
    return weight_bytes(encoding, n, k) + x_itemsize * m * k + out_itemsize * m * n


def copies_for(bytes_per_rotation_unit):
    return max(2, math.ceil(ROTATION_BYTES / bytes_per_rotation_unit))


# ------------------------------------------------------------------ timing --

TIMING = "graph"    # --timing
WARM_SECONDS = 0.1  # --warm-seconds


def warm(device, run):
    """Call ``run`` (which enqueues GPU work) back to back until WARM_SECONDS have passed."""
    start = time.perf_counter()
    while True:
        run()
        device.synchronize()
        if time.perf_counter() - start >= WARM_SECONDS:
            return


def summarize(samples_s, per):
    """Per-unit statistics of replay samples (seconds per replay, ``per`` units per replay)."""
    us = [s / per * 1e6 for s in samples_s]
    return {"median_us": round(statistics.median(us), 3), "min_us": round(min(us), 3),
            "max_us": round(max(us), 3), "samples_us": [round(u, 3) for u in us]}


def time_launches(device, launches, per=1, replays=REPLAYS):
    """Time one pass over ``launches`` (callables that enqueue work): replayed from one
    captured HIP graph (``--timing graph``) or enqueued eagerly (``--timing eager``), each
    replay bracketed by HIP events on the launch stream.  Returns per-unit statistics."""
    def timed(run):
        samples = []
        for _ in range(replays):
            start = device.record_event(timing=True)
            run()
            stop = device.record_event(timing=True)
            stop.synchronize()
            samples.append(device.elapsed_ms(start, stop) * 1e-3)
            start.release()
            stop.release()
        return samples

    if TIMING == "eager":
        def run():
            for launch in launches:
                launch()
        warm(device, run)
        return summarize(timed(run), per)
    graph = device.graph(lambda: [launch() for launch in launches])
    try:
        warm(device, graph.replay)
        return summarize(timed(graph.replay), per)
    finally:
        graph.close()


def rate(stats, work, unit):
    """Throughput at the median (and the spread in the same unit) for ``work`` per unit."""
    scale = 1e-3 if unit == "GB/s" else 1e-6  # bytes/us -> GB/s; flops/us -> TFLOP/s
    return {unit: round(work / stats["median_us"] * scale, 2),
            f"{unit}_best": round(work / stats["min_us"] * scale, 2)}


# ------------------------------------------------------------------ layers --

def rotated(device, raw, copies):
    first = device.from_numpy(raw)
    return [first] + [device.empty(raw.shape, "uint8").copy_from(first) for _ in range(copies - 1)]


class Linear:
    """One linear layer: rotated weight copies, its input and output, bound calls."""

    def __init__(self, device, kernel, encoding, m, n, k, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        self.m, self.n, self.k = m, n, k
        self.weights = rotated(device, cases.weight(n, k, encoding, seed), copies)
        self.owned = [] if x is not None else [device.from_numpy(cases.activation(m, k, seed + 1))]
        self.x = x if x is not None else self.owned[0]
        self.out = device.empty((m, n), out_dtype)
        exe = device.load(kernel, encoding=encoding, out_dtype=out_dtype)
        self.calls = [exe.bind(self.x, w, self.out) for w in self.weights]
        self.bytes = gemv_bytes(encoding, m, n, k, np.dtype(out_dtype).itemsize)
        self.flops = 2 * m * n * k

    def release(self):
        for b in self.weights + [self.out] + self.owned:
            b.release()


class GroupLinear:
    """Matrices sharing one activation input, launched as one grouped GEMV call."""

    def __init__(self, device, encoding, m, shapes, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        k = shapes[0][1]
        assert all(sk == k for _, sk in shapes)
        self.weights = [rotated(device, cases.weight(n, k, encoding, seed + 2 * i), copies)
                        for i, (n, _) in enumerate(shapes)]
        self.owned = [] if x is not None else [device.from_numpy(cases.activation(m, k, seed + 1))]
        self.x = x if x is not None else self.owned[0]
        self.outs = [device.empty((m, n), out_dtype) for n, _ in shapes]
        exe = device.load("gguf_gemv_group", encoding=encoding, out_dtype=out_dtype, count=len(shapes))
        self.calls = []
        for c in range(copies):
            args = [self.x]
            for ws, out in zip(self.weights, self.outs):
                args += [ws[c], out]
            self.calls.append(exe.bind(*args))
        itemsize = np.dtype(out_dtype).itemsize
        self.bytes = sum(weight_bytes(encoding, n, k) + itemsize * m * n for n, _ in shapes) + 2 * m * k
        self.flops = sum(2 * m * n * k for n, _ in shapes)

    def release(self):
        for b in [w for ws in self.weights for w in ws] + self.outs + self.owned:
            b.release()


class SwigluLinear:
    """An MLP's gate and up matrices launched as one SwiGLU GEMV: out = silu(x Wg^T) * (x Wu^T)."""

    def __init__(self, device, encoding, m, n, k, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        self.weights = [rotated(device, cases.weight(n, k, encoding, seed + 2 * i), copies) for i in range(2)]
        self.owned = [] if x is not None else [device.from_numpy(cases.activation(m, k, seed + 1))]
        self.x = x if x is not None else self.owned[0]
        self.out = device.empty((m, n), out_dtype)
        exe = device.load("gguf_gemv_swiglu", encoding=encoding, out_dtype=out_dtype)
        self.calls = [exe.bind(self.x, self.weights[0][c], self.weights[1][c], self.out) for c in range(copies)]
        self.bytes = 2 * weight_bytes(encoding, n, k) + 2 * m * k + np.dtype(out_dtype).itemsize * m * n
        self.flops = 4 * m * n * k

    def release(self):
        for b in [w for ws in self.weights for w in ws] + [self.out] + self.owned:
            b.release()


class GroupGemm:
    """Prefill GEMM of matrices sharing one activation input (gguf_gemm_group), rotated weight
    copies, on a workspace the caller provides (shared by launches that run one at a time)."""

    def __init__(self, device, encoding, m, k, rows, out_dtype, copies, seed, workspace):
        from tests import gguf_cases as cases

        self.weights = [rotated(device, cases.weight(n, k, encoding, seed + i), copies) for i, n in enumerate(rows)]
        self.x = device.from_numpy(cases.activation(m, k, seed + 10))
        self.outs = [device.empty((m, n), out_dtype) for n in rows]
        exe = device.load("gguf_gemm_group", encoding=encoding, out_dtype=out_dtype, count=len(rows))
        self.calls = []
        for c in range(copies):
            args = [self.x]
            for ws, out in zip(self.weights, self.outs):
                args += [ws[c], out]
            self.calls.append(exe.bind(*args, workspace))
        self.flops = sum(2 * m * n * k for n in rows)

    def release(self):
        for b in [w for ws in self.weights for w in ws] + self.outs + [self.x]:
            b.release()


def rotated_launches(linears, steps):
    """``steps`` passes over the linears, each pass using the next weight copy."""
    return [layer.calls[step % len(layer.calls)].launch for step in range(steps) for layer in linears]


# -------------------------------------------------------- committed profile --

PROFILE = os.path.join(ROOT, "profiles", "gemv_q4k_m1_qwen3_mlp.md")


def profile_figures():
    """Machine-readable lines of the committed rocprofv3 summary of the roofline kernel:
    ``traffic_bytes_per_launch`` (FETCH_SIZE / WRITE_SIZE passes scaled by a 256 MiB copy)
    and ``avg_us_per_launch`` (kernel-trace average); empty if the file is absent."""
    figures = {}
    try:
        with open(PROFILE) as f:
            for line in f:
                key, sep, value = line.partition(":")
                if sep and key in ("traffic_bytes_per_launch", "avg_us_per_launch"):
                    figures[key] = float(value)
    except OSError:
        pass
    return figures


# ------------------------------------------------------------ CPU baseline --

def cpu_threads():
    """Threads for the all-cores leg: the CPUs this process may run on, capped by the job's CPU
    share (OMP_NUM_THREADS, set to the share on the GPU boxes)."""
    available = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    return (min(available, int(share)) if share and share.isdigit() and int(share) > 0 else available), available


CPU_DTYPE_IDS = {np.dtype(np.float16): 10, np.dtype(np.float32): 11, np.dtype(np.uint8): 3}


def cpu_call(x, raw, out, code):
    """A TensorCallV1 for the oracle's CPU entries over host arrays [x, w, out, type], built as
    the reference CPU provider builds one for a native image (src/tensor/providers/cpu.py:153-197).
    Returns (call, keep): ``keep`` holds the shape / stride arrays the descriptor points at."""
    import ctypes as c

    from tensor_amd.runtime import abi

    keep, args = [], (abi.Argument * 4)()
    for j, arr in enumerate((x, raw, out)):
        shape = (c.c_int64 * 2)(*arr.shape)
        strides = (c.c_int64 * 2)(arr.strides[0], arr.strides[1])
        keep += [shape, strides, arr]
        dtype = CPU_DTYPE_IDS[arr.dtype]
        args[j].kind, args[j].dtype = 1, dtype
        args[j].buffer = abi.BufferDescriptor(arr.ctypes.data, arr.nbytes, shape, strides, 2, dtype, 1, 0)
    args[3].kind, args[3].dtype, args[3].scalar = 2, 7, code
    call = abi.CallDescriptor(1, 72, args, 4, 0, (c.c_uint32 * 3)(1, 1, 1), (c.c_uint32 * 3)(1, 1, 1), 0,
                              abi.StreamDescriptor(1, 0, 0))
    keep.append(args)
    return call, keep


def cpu_baseline(budget_s=20.0):
    """Time the oracle's TensorKernelV1 CPU entries, invoked as the reference CPU provider
    invokes a native image (ctypes, synchronous call; src/tensor/providers/cpu.py:153-197):
    tensor_gguf_gemv_cpu_v1 (decode numerics) on the headline step, C1, C2 at M = 4 / 8, C3 and
    C5 at M = 1, and tensor_gguf_gemm_cpu_v1 (prefill numerics: fp16 operands, fp32
    accumulation) on C4 at M = 512 / 2048 and C5 at M = 256.  Every config reports all-core and
    single-thread figures; where a full call would take minutes the timed call covers a
    stated slice of the weight rows (rows are independent, so the rate is the config's)."""
    import ctypes as c

    from oracle import gguf_ref
    from tensor_amd.runtime import abi
    from tests import gguf_cases as cases

    if not gguf_ref.LIBRARY.exists():
        gguf_ref.build()
    oracle = gguf_ref.c_oracle()
    for entry in (oracle.entry, oracle.gemm_entry):
        entry.argtypes = [c.POINTER(abi.CallDescriptor), c.POINTER(abi.ErrorDescriptor)]
        entry.restype = c.c_int32
    threads, available = cpu_threads()
    codes = {"q8_0": 8, "q4_k": 12, "q6_k": 14}

    def layers_for(shapes, m, out_dtype, seed, rotate=True):
        """Bound CPU calls for each (encoding, n, k), weights rotated past the host LLC."""
        step_weights = sum(weight_bytes(e, n, k) for e, n, k in shapes)
        copies = 1 if not rotate or step_weights >= 256 * 2**20 else math.ceil(512 * 2**20 / step_weights)
        out = []
        for i, (encoding, n, k) in enumerate(shapes):
            first = cases.weight(n, k, encoding, seed + i)
            x = cases.activation(m, k, seed + 100 + i)
            o = np.empty((m, n), out_dtype)
            out.append([cpu_call(x, first if r == 0 else first.copy(), o, codes[encoding]) for r in range(copies)])
        return out, copies

    def measure(entry, calls, threads_, seconds, at_least=3):
        oracle.set_threads(threads_)
        error = abi.ErrorDescriptor()
        samples, step, begin = [], 0, time.perf_counter()
        while time.perf_counter() - begin < seconds or len(samples) < at_least:
            t0 = time.perf_counter()
            for layer in calls:
                if entry(c.byref(layer[step % len(layer)][0]), c.byref(error)):
                    raise RuntimeError(error.message.decode())
            samples.append(time.perf_counter() - t0)
            step += 1
        return statistics.median(samples), len(samples)

    def config(name, shapes, m, out_dtype, seconds, seed, gemm=False, slices=(1, 1)):
        """``slices`` = (all-core, single-thread) divisors of each matrix's rows for the timed calls."""
        entry = oracle.gemm_entry if gemm else oracle.entry
        itemsize = np.dtype(out_dtype).itemsize
        result = {"numerics": "prefill: fp16 x . fp16(dequant W), fp32 accumulate" if gemm else
                  "decode: fp32 x . fp32 dequant W, fp32 accumulate"}
        for label, threads_, divisor, budget in (("", threads, slices[0], seconds), ("single_thread_", 1, slices[1],
                                                                                     seconds / 2)):
            sample = [(e, n // divisor, k) for e, n, k in shapes]
            calls, copies = layers_for(sample, m, out_dtype, seed, rotate=not gemm)
            nbytes = sum(gemv_bytes(e, m, n, k, itemsize) for e, n, k in sample)
            flops = sum(2 * m * n * k for _, n, k in sample)
            seconds_per_call, count = measure(entry, calls, threads_, budget, at_least=1 if label else 3)
            full = seconds_per_call * divisor
            result.update({f"{label}ms": round(full * 1e3, 3), f"{label}calls": count,
                           f"{label}GB/s": round(nbytes / seconds_per_call / 1e9, 3),
                           f"{label}GFLOP/s": round(flops / seconds_per_call / 1e9, 3)})
            if divisor > 1:
                result[f"{label}sample"] = f"1/{divisor} of each matrix's rows per call; ms scaled to the full call"
            if not label:
                result.update(threads=threads, weight_copies=copies)
        log("cpu", name, result)
        return result

    share = budget_s / 10.0
    layer_shapes = [("q4_k", 4096, 4096), ("q4_k", 1024, 4096), ("q4_k", 1024, 4096), ("q4_k", 4096, 4096),
                    ("q4_k", 12288, 4096), ("q4_k", 12288, 4096), ("q6_k", 4096, 12288)]
    per_config = {
        "C1_q8_0_gemv_m1_4096x4096": config("C1", [("q8_0", 4096, 4096)], 1, np.float16, share, 3000),
        "C2_q4k_gemv_m4_12288x4096": config("C2 M=4", [("q4_k", 12288, 4096)], 4, np.float16, share, 3100),
        "C2_q4k_gemv_m8_12288x4096": config("C2 M=8", [("q4_k", 12288, 4096)], 8, np.float16, share, 3200),
        "C3_q6k_lm_head_m1_151936x4096_fp32": config("C3", [("q6_k", 151936, 4096)], 1, np.float32, share, 3300),
        "C4_q4k_gemm_m512_12288x4096": config("C4 M=512", [("q4_k", 12288, 4096)], 512, np.float16, share, 3500,
                                              gemm=True, slices=(1, 16)),
        "C4_q4k_gemm_m2048_12288x4096": config("C4 M=2048", [("q4_k", 12288, 4096)], 2048, np.float16, share,
                                               3600, gemm=True, slices=(4, 64)),
        "C5_layer_m1": config("C5 M=1", layer_shapes, 1, np.float16, share, 3400),
        "C5_layer_m256": config("C5 M=256", layer_shapes, 256, np.float16, share, 3700, gemm=True,
                                slices=(2, 32)),
    }
    headline_shapes = [("q4_k", 12288, 4096), ("q4_k", 12288, 4096), ("q4_k", 4096, 12288)]
    calls, copies = layers_for(headline_shapes, 1, np.float16, 1000)
    step_bytes = sum(gemv_bytes(e, 1, n, k, 2) for e, n, k in headline_shapes)
    multi, n_multi = measure(oracle.entry, calls, threads, budget_s * 0.3)
    single, n_single = measure(oracle.entry, calls, 1, budget_s * 0.2)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(step_bytes / multi / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n_multi} headline steps (Q4_K GEMV M=1 gate+up+down, {step_bytes} B/step), median "
                  f"{multi * 1e3:.2f} ms/step on {threads} threads; weights rotated over {copies} copies",
        "single_thread_gbs": round(step_bytes / single / 1e9, 3),
        "single_thread_ms_per_step": round(single * 1e3, 3),
        "cores_available": available,
        "cores_note": "threads = the CPUs this process may use, capped by the job's CPU share (OMP_NUM_THREADS)",
        "cpu_model": model,
        "per_config": per_config,
    }


# -------------------------------------------------------------- torch leg --

def torch_leg():
    """The reference's resident-dequantized lower bound (benchmark.py:478-488): torch.mm in fp16
    on weights already dequantized and resident in HBM, at the prefill and showcase shapes,
    timed with this file's graph protocol.  Runs in its own process, torch imported first, and
    prints one JSON object.  Weights are seeded N(0, 0.02) in fp16 (torch.mm's time does not
    depend on the values); the right operand is a contiguous [K, N] copy of W^T."""
    import torch

    assert torch.cuda.is_available()
    device = torch.device("cuda")
    results = {}

    def graph_time(call, iterations):
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iterations):
                call()
        start = time.perf_counter()
        while time.perf_counter() - start < WARM_SECONDS:
            graph.replay()
            torch.cuda.synchronize()
        samples = []
        for _ in range(REPLAYS):
            begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            begin.record()
            graph.replay()
            end.record()
            end.synchronize()
            samples.append(begin.elapsed_time(end) * 1e-3)
        del graph
        return summarize(samples, iterations)

    gen = torch.Generator(device="cpu").manual_seed(5)
    for name, m, n, k in (("C4_m512_12288x4096", 512, 12288, 4096), ("C4_m2048_12288x4096", 2048, 12288, 4096),
                          ("C5_m256_q_4096x4096", 256, 4096, 4096), ("C5_m256_k_1024x4096", 256, 1024, 4096),
                          ("C5_m256_gate_12288x4096", 256, 12288, 4096), ("C5_m256_down_4096x12288", 256, 4096, 12288)):
        x = torch.randn(m, k, generator=gen).half().to(device)
        w_t = (torch.randn(k, n, generator=gen) * 0.02).half().to(device)  # W^T, [K, N], contiguous
        out = torch.empty(m, n, dtype=torch.float16, device=device)
        stats = graph_time(lambda: torch.mm(x, w_t, out=out), 10)
        results[name] = dict(stats, **rate(stats, 2 * m * n * k, "TFLOP/s"))
        print(f"[torch-leg] {name} {stats['median_us']} us", file=sys.stderr, flush=True)
        del x, w_t, out
    for m in (1, 32):  # the showcase's own baseline: fp32 x -> fp16, mm, -> fp32 out
        n = k = 1024
        x32 = torch.randn(m * k, generator=gen).to(device) * 0.2
        w_t = (torch.randn(k, n, generator=gen) * 0.02).half().to(device)
        activation = torch.empty(m, k, dtype=torch.float16, device=device)
        temp = torch.empty(m, n, dtype=torch.float16, device=device)
        out = torch.empty(m * n, dtype=torch.float32, device=device)

        def baseline():
            activation.copy_(x32.reshape(m, k))
            torch.mm(activation, w_t, out=temp)
            out.copy_(temp.reshape(-1))

        stats = graph_time(baseline, 30)
        results[f"showcase_m{m}_1024x1024"] = stats
        print(f"[torch-leg] showcase m={m} {stats['median_us']} us", file=sys.stderr, flush=True)
    print(json.dumps({"torch": torch.__version__, "hip": torch.version.hip, "cases": results}))


def run_torch_leg():
    """Run torch_leg() in a child process (torch must own the process's HIP runtime)."""
    command = [sys.executable, "-u", os.path.abspath(__file__), "--torch-leg", "--warm-seconds", str(WARM_SECONDS)]
    try:
        done = subprocess.run(command, capture_output=True, text=True, timeout=600, cwd=ROOT)
    except subprocess.TimeoutExpired:
        return {"error": "torch leg timed out"}
    sys.stderr.write(done.stderr[-3000:])
    if done.returncode:
        return {"error": f"torch leg exited with {done.returncode}"}
    return json.loads(done.stdout.strip().splitlines()[-1])


# ---------------------------------------------------------------- details --

def detail_cases(device):
    """(name, function) for every details case; each builds, times and releases its own buffers."""
    from tests import gguf_cases as cases

    cases_ = []

    def add(name):
        def register(function):
            cases_.append((name, function))
            return function
        return register

    def gemv_case(name, encoding, m, n, k, out_dtype, launches=60):
        @add(name)
        def run():
            copies = copies_for(weight_bytes(encoding, n, k))
            layer = Linear(device, "gguf_gemv", encoding, m, n, k, out_dtype, copies, 7 + m)
            stats = time_launches(device, [layer.calls[i % copies].launch for i in range(launches)], per=launches)
            result = dict(stats, **rate(stats, layer.bytes, "GB/s"), copies=copies)
            result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
            layer.release()
            return result

    def mlp_copies():
        return copies_for(2 * weight_bytes("q4_k", 12288, 4096) + weight_bytes("q4_k", 4096, 12288))

    @add("C2_step_m1_three_launches")
    def three_launches():
        copies = mlp_copies()
        x = device.from_numpy(cases.activation(1, 4096, 2))
        mlp = [Linear(device, "gguf_gemv", "q4_k", 1, 12288, 4096, "float16", copies, 1, x=x),
               Linear(device, "gguf_gemv", "q4_k", 1, 12288, 4096, "float16", copies, 3, x=x),
               Linear(device, "gguf_gemv", "q4_k", 1, 4096, 12288, "float16", copies, 5)]
        stats = time_launches(device, rotated_launches(mlp, 50), per=50)
        result = dict(stats, **rate(stats, sum(layer.bytes for layer in mlp), "GB/s"))
        result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
        for layer in mlp:
            layer.release()
        x.release()
        return result

    @add("C2_step_m1_swiglu")
    def swiglu_step():
        # the MLP as a decode step runs it: gate + up with the SwiGLU epilogue in one launch,
        # then down on its output
        copies = mlp_copies()
        fused = SwigluLinear(device, "q4_k", 1, 12288, 4096, "float16", copies, 60)
        down = Linear(device, "gguf_gemv", "q4_k", 1, 4096, 12288, "float16", copies, 64, x=fused.out)
        stats = time_launches(device, rotated_launches([fused, down], 50), per=50)
        result = dict(stats, **rate(stats, fused.bytes + down.bytes, "GB/s"), launches=2)
        result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
        down.release()
        fused.release()
        return result

    for m in (1, 4, 8):
        @add(f"C2_q4k_gemv_swiglu_m{m}_12288x4096")
        def swiglu_pair(m=m):
            copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096))
            pair = SwigluLinear(device, "q4_k", m, 12288, 4096, "float16", copies, 66 + m)
            stats = time_launches(device, [pair.calls[i % copies].launch for i in range(60)], per=60)
            result = dict(stats, **rate(stats, pair.bytes, "GB/s"), copies=copies)
            result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
            pair.release()
            return result

    for m in (4, 8):
        @add(f"C2_q4k_gemv_group_m{m}_2x12288x4096")
        def group_pair(m=m):
            copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096))
            group = GroupLinear(device, "q4_k", m, [(12288, 4096), (12288, 4096)], "float16", copies, 70 + m)
            stats = time_launches(device, [group.calls[i % copies].launch for i in range(60)], per=60)
            result = dict(stats, **rate(stats, group.bytes, "GB/s"), copies=copies)
            result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
            group.release()
            return result

    @add("C2_host_enqueue_m1_gate_up")
    def host_enqueue():
        # host cost of one eager launch of the headline's grouped gate + up GEMV through
        # BoundCall.launch (tensor.runtime.bench's three figures; src/tensor/runtime/timing.py:10-43)
        from tensor_amd.runtime.timing import bench as runtime_bench

        group = GroupLinear(device, "q4_k", 1, [(12288, 4096), (12288, 4096)], "float16", 1, 80)
        exe = device.load("gguf_gemv_group", encoding="q4_k", out_dtype="float16", count=2)
        figures = runtime_bench(exe, (group.x, group.weights[0][0], group.outs[0], group.weights[1][0], group.outs[1]),
                                warmup=50, iters=200)
        group.release()
        return {"host_enqueue_us": round(figures["median_host_enqueue_seconds"] * 1e6, 2),
                "launch_and_sync_us": round(figures["median_launch_and_sync_seconds"] * 1e6, 2),
                "device_us": round(figures["median_device_seconds"] * 1e6, 3),
                "timing": "tensor_amd.runtime.timing.bench: medians of 200 eager launches, one weight copy"}

    # C1's shape (the reference runs it on its CPU provider) on the GPU
    gemv_case("C1_q8_0_gemv_m1_4096x4096", "q8_0", 1, 4096, 4096, "float16")
    gemv_case("C5_q6k_gemv_m1_4096x12288", "q6_k", 1, 4096, 12288, "float16")
    for m in (1, 4, 8):
        gemv_case(f"C2_q4k_gemv_m{m}_12288x4096", "q4_k", m, 12288, 4096, "float16")
        gemv_case(f"C2_q4k_gemv_m{m}_4096x12288", "q4_k", m, 4096, 12288, "float16")
    gemv_case("C3_q6k_lm_head_m1_151936x4096_fp32", "q6_k", 1, 151936, 4096, "float32")
    # one GPU's share of an 8-way tensor-parallel decode step: column-parallel gate (and up)
    # rows, the row-parallel down's K slice (its partial sums would then be all-reduced), the
    # vocab-parallel LM head
    gemv_case("shard8_q4k_gate_m1_1536x4096", "q4_k", 1, 1536, 4096, "float16")
    gemv_case("shard8_q4k_down_m1_4096x1536", "q4_k", 1, 4096, 1536, "float16")
    gemv_case("shard8_q6k_down_m1_4096x1536", "q6_k", 1, 4096, 1536, "float16")
    gemv_case("shard8_q6k_lm_head_m1_18992x4096_fp32", "q6_k", 1, 18992, 4096, "float32")
    for encoding in ("q6_k", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q5_k"):
        gemv_case(f"enc_{encoding}_gemv_m1_12288x4096", encoding, 1, 12288, 4096, "float16")

    def gemm_case(name, encoding, m, n, k, launches=10):
        @add(name)
        def run():
            layer = Linear(device, "gguf_gemm", encoding, m, n, k, "float16", 2, 9)
            stats = time_launches(device, [layer.calls[i % 2].launch for i in range(launches)], per=launches)
            result = dict(stats, **rate(stats, layer.flops, "TFLOP/s"))
            result["mfma_frac"] = round(result["TFLOP/s"] / FP16_PEAK_TFLOPS, 4)
            layer.release()
            return result

    gemm_case("C4_q4k_gemm_m512_12288x4096", "q4_k", 512, 12288, 4096)
    gemm_case("C4_q4k_gemm_m2048_12288x4096", "q4_k", 2048, 12288, 4096, launches=4)
    for encoding in ("q5_k", "q8_0", "q4_0"):
        gemm_case(f"enc_{encoding}_gemm_m512_12288x4096", encoding, 512, 12288, 4096)

    # C5: q, k, v, o, gate, up (Q4_K) and down (Q6_K) chained on one stream
    shapes = [("q", "q4_k", 4096, 4096), ("k", "q4_k", 1024, 4096), ("v", "q4_k", 1024, 4096),
              ("o", "q4_k", 4096, 4096), ("gate", "q4_k", 12288, 4096), ("up", "q4_k", 12288, 4096),
              ("down", "q6_k", 4096, 12288)]
    layer_weights = sum(weight_bytes(e, n, k) for _, e, n, k in shapes)
    def layer_prefill(m):
        # the prefill step: q + k + v and gate + up as grouped GEMMs, o, then down, each on the
        # plan the library picks (K split across workgroups for q + k + v and the Q6_K down at
        # M=256; at M=32 and 128 the small- and mid-M plans); below M=256 the weights rotate
        # through enough copies to stay out of the MALL, since the launches then stream them
        groups = [("qkv", "q4_k", 4096, [4096, 1024, 1024]), ("o", "q4_k", 4096, [4096]),
                  ("gate_up", "q4_k", 4096, [12288, 12288]), ("down", "q6_k", 12288, [4096])]
        need = max(device.gemm_workspace(e, m, k, rows) for _, e, k, rows in groups)
        workspace = device.empty((max(need, 256),), "uint8")
        copies = 2 if m >= 256 else copies_for(layer_weights)
        layers = [GroupGemm(device, e, m, k, rows, "float16", copies, 30 + 5 * i, workspace)
                  for i, (_, e, k, rows) in enumerate(groups)]
        steps = max(4, copies)
        stats = time_launches(device, rotated_launches(layers, steps), per=steps)
        result = dict(stats, **rate(stats, sum(layer.flops for layer in layers), "TFLOP/s"), launches=len(layers),
                      workspace_bytes=need)
        result["mfma_frac"] = round(result["TFLOP/s"] / FP16_PEAK_TFLOPS, 4)
        result["per_group_us"] = {}
        for (name, *_), layer in zip(groups, layers):
            one = time_launches(device, [layer.calls[i % copies].launch for i in range(10)], per=10)
            result["per_group_us"][name] = one["median_us"]
        for layer in layers:
            layer.release()
        workspace.release()
        return result

    add("C5_layer_m256")(lambda: layer_prefill(256))
    add("C5_layer_m128_grouped")(lambda: layer_prefill(128))
    add("C5_layer_m32_grouped")(lambda: layer_prefill(32))

    for m, kernel in ((1, "gguf_gemv"), (256, "gguf_gemm")):
        @add(f"C5_layer_m{m}" if m == 1 else "C5_layer_m256_seven_launches")
        def layer_chain(m=m, kernel=kernel):
            copies = copies_for(layer_weights) if m == 1 else 2
            layers = [Linear(device, kernel, e, m, n, k, "float16", copies, 20 + i)
                      for i, (_, e, n, k) in enumerate(shapes)]
            steps = 20 if m == 1 else 4
            stats = time_launches(device, rotated_launches(layers, steps), per=steps)
            result = dict(stats, **rate(stats, sum(layer.bytes for layer in layers), "GB/s"),
                          **rate(stats, sum(layer.flops for layer in layers), "TFLOP/s"))
            if m > 1:  # each linear on its own, for the per-kernel picture
                result["per_linear_us"] = {}
                for (name, *_), layer in zip(shapes, layers):
                    one = time_launches(device, [layer.calls[i % 2].launch for i in range(10)], per=10)
                    result["per_linear_us"][name] = one["median_us"]
            for layer in layers:
                layer.release()
            return result

    @add("C5_layer_m1_grouped")
    def layer_grouped():
        # C5 at M=1 the way a decode step runs it: q + k + v grouped, o, gate + up grouped, down
        copies = copies_for(layer_weights)
        x = device.from_numpy(np.zeros((1, 4096), np.float16) + np.float16(0.5))
        layers = [GroupLinear(device, "q4_k", 1, [(4096, 4096), (1024, 4096), (1024, 4096)], "float16", copies, 40,
                              x=x),
                  Linear(device, "gguf_gemv", "q4_k", 1, 4096, 4096, "float16", copies, 46, x=x),
                  GroupLinear(device, "q4_k", 1, [(12288, 4096), (12288, 4096)], "float16", copies, 48, x=x),
                  Linear(device, "gguf_gemv", "q6_k", 1, 4096, 12288, "float16", copies, 52)]
        stats = time_launches(device, rotated_launches(layers, 20), per=20)
        result = dict(stats, **rate(stats, sum(layer.bytes for layer in layers), "GB/s"), launches=4)
        for layer in layers:
            layer.release()
        x.release()
        return result

    # The showcase's packed call form (fp32 x and out) at the BASELINE decode shapes, weights
    # rotated out of the MALL: the cost of the fp32-activation path against the fp16 cases above
    for encoding, n, k in (("q8_0", 4096, 4096), ("q4_k", 12288, 4096), ("q4_k", 4096, 12288),
                           ("q6_k", 151936, 4096)):
        @add(f"packed_{encoding}_m1_{n}x{k}_fp32x")
        def packed_decode(encoding=encoding, n=n, k=k):
            copies = copies_for(weight_bytes(encoding, n, k))
            x = device.from_numpy(cases.activation(1, k, 5).astype(np.float32).reshape(-1))
            weights = rotated(device, cases.weight(n, k, encoding, 6).reshape(-1), copies)
            out = device.empty((n,), "float32")
            exe = device.load("gguf_linear", encoding=encoding, m=1, n=n, k=k)
            calls = [exe.bind(x, w, out) for w in weights]
            stats = time_launches(device, [calls[i % copies].launch for i in range(60)], per=60)
            result = dict(stats, **rate(stats, gemv_bytes(encoding, 1, n, k, 4, 4), "GB/s"), copies=copies)
            result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
            for b in [x, out, *weights]:
                b.release()
            return result

    # The Q8_1-activation integer-dot GEMV (GGML's path; fp32 x quantized in each workgroup,
    # fp16 out) at BASELINE decode shapes, weights rotated: beside the fp32-decode kernels above
    for encoding, m, n, k in (("q8_0", 1, 4096, 4096), ("q4_k", 1, 12288, 4096), ("q6_k", 1, 4096, 12288),
                              ("q4_k", 4, 12288, 4096), ("q4_k", 8, 12288, 4096)):
        @add(f"q8_1_{encoding}_m{m}_{n}x{k}")
        def q8_1_decode(encoding=encoding, m=m, n=n, k=k):
            copies = copies_for(weight_bytes(encoding, n, k))
            x = device.from_numpy(cases.activation(m, k, 5).astype(np.float32))
            weights = rotated(device, cases.weight(n, k, encoding, 6), copies)
            out = device.empty((m, n), "float16")
            exe = device.load("gguf_gemv_q8_1", encoding=encoding, out_dtype="float16", x_dtype="float32")
            calls = [exe.bind(x, w, out) for w in weights]
            stats = time_launches(device, [calls[i % copies].launch for i in range(60)], per=60)
            result = dict(stats, **rate(stats, gemv_bytes(encoding, m, n, k, 2, 4), "GB/s"), copies=copies)
            result["hbm_frac"] = round(result["GB/s"] / HBM_PEAK_GBS, 4)
            for b in [x, out, *weights]:
                b.release()
            return result

    # The showcase's packed call at its own shapes (N = K = 1024, M in {1, 32}, fp32 x and out,
    # benchmark.py:122-126, :460-464), hot-cache as the reference times it (one weight copy).
    for encoding in ("q4_0", "q4_k", "q6_k"):
        for m in (1, 32):
            @add(f"showcase_{encoding}_m{m}_1024x1024")
            def showcase(encoding=encoding, m=m):
                n = k = 1024
                x = (np.random.default_rng(m).standard_normal(m * k, dtype=np.float32) * np.float32(0.2))
                xb = device.from_numpy(x)
                wb = device.from_numpy(cases.weight(n, k, encoding, 11).reshape(-1))
                out = device.empty((m * n,), "float32")
                call = device.load("gguf_linear", encoding=encoding, m=m, n=n, k=k).bind(xb, wb, out)
                stats = time_launches(device, [call.launch] * 30, per=30)
                result = dict(stats, **rate(stats, gemv_bytes(encoding, m, n, k, 4, 4), "GB/s"),
                              **rate(stats, 2 * m * n * k, "TFLOP/s"))
                result["l4_reference_us"] = L4_SHOWCASE_US[(encoding, m)]
                for b in (xb, wb, out):
                    b.release()
                return result

    return cases_


def run_details(device, only=None):
    """Every details case whose name starts with ``only`` (all by default), in a seeded shuffled
    order (benchmark.py:1007-1013 shuffles its providers with random.Random(42))."""
    chosen = [(name, run) for name, run in detail_cases(device) if only is None or name.startswith(only)]
    random.Random(42).shuffle(chosen)
    details = {"measurement_order": [name for name, _ in chosen]}
    for name, run in chosen:
        details[name] = run()
        log(name, {k: v for k, v in details[name].items() if k != "samples_us"})
    return details


# ------------------------------------------------------------- plan sweep --

SWEEP_SHAPES = (("C4_q4k_m512_12288x4096", "q4_k", 512, 4096, (12288,)),
                ("C4_q4k_m2048_12288x4096", "q4_k", 2048, 4096, (12288,)),
                ("C5_m256_qkv", "q4_k", 256, 4096, (4096, 1024, 1024)),
                ("C5_m256_o", "q4_k", 256, 4096, (4096,)),
                ("C5_m256_gate_up", "q4_k", 256, 4096, (12288, 12288)),
                ("C5_m256_down_q6k", "q6_k", 256, 12288, (4096,)))
SWEEP_SPLITS = (1, 2, 4, 8)
SWEEP_WORKSPACE = 256 << 20  # plans whose partial sums need more are not candidates


def plan_sweep(device, only=None):
    """Every plan of the pipelined prefill GEMM (tile x K split) at the BASELINE GEMM shapes,
    timed, then the three fastest re-timed on their own before the winner is named, as the
    reference's schedule search does (benchmarks/kernels/showcase/benchmark.py:214-237, :917-932);
    beside the winner, the plan the library picks.  Each candidate's output is checked against the
    library plan's (rel-L2 <= 2e-3, no NaN) before it is timed."""
    from oracle import gguf_ref as R
    from tensor_amd.providers.hip import gemm_tiles
    from tests import gguf_cases as cases

    tiles = gemm_tiles()
    report = {}
    for name, encoding, m, k, rows in SWEEP_SHAPES:
        if only is not None and not name.startswith(only):
            continue
        chosen = device.gemm_plan(encoding, m, k, rows)
        weights = [device.from_numpy(cases.weight(n, k, encoding, 1200 + i)) for i, n in enumerate(rows)]
        x = device.from_numpy(cases.activation(m, k, 1210))
        outs = [device.empty((m, n), "float16") for n in rows]
        workspace = device.empty((SWEEP_WORKSPACE,), "uint8")
        exe = device.load("gguf_gemm_group_plan", encoding=encoding, out_dtype="float16", count=len(rows))
        args = [x]
        for w, out in zip(weights, outs):
            args += [w, out]
        flops = sum(2 * m * n * k for n in rows)

        def run_plan(tile, splits):
            return exe.bind(*args, workspace, tile=tile, splits=splits)

        reference = run_plan(chosen["tile"], chosen["splits"]) if chosen["pipelined"] else None
        expected = None
        if reference is not None:
            reference.launch()
            expected = [out.to_numpy().astype(np.float32) for out in outs]
        candidates = []
        for tile, geometry in enumerate(tiles):
            for splits in SWEEP_SPLITS:
                if splits * m * sum(rows) * 4 > SWEEP_WORKSPACE and splits > 1:
                    continue
                try:
                    call = run_plan(tile, splits)
                    for out in outs:
                        device.fill_bytes(out, 0xFF)
                    call.launch()
                except Exception as exc:  # the entry refuses plans that do not fit the shape
                    if getattr(exc, "code", None) == 2:
                        continue
                    raise
                got = [out.to_numpy().astype(np.float32) for out in outs]
                ok = all(not np.isnan(g).any() for g in got)
                if ok and expected is not None:
                    ok = max(R.relative_l2(g, e) for g, e in zip(got, expected)) <= 2e-3
                stats = time_launches(device, [call.launch] * 10, per=10, replays=5)
                candidates.append({"tile": tile, **geometry, "splits": splits, "valid": bool(ok),
                                   "median_us": stats["median_us"], "call": call})
        finalists = sorted((c for c in candidates if c["valid"]), key=lambda c: c["median_us"])[:3]
        for c in finalists:
            c["selection"] = time_launches(device, [c["call"].launch] * 60, per=60, replays=7)
        winner = min(finalists, key=lambda c: c["selection"]["median_us"])
        library = next((c for c in candidates if (c["tile"], c["splits"]) == (chosen["tile"], chosen["splits"])), None)
        if library is not None and "selection" not in library:
            library["selection"] = time_launches(device, [library["call"].launch] * 60, per=60, replays=7)

        def public(c):
            out = {key: value for key, value in c.items() if key != "call"}
            if "selection" in c:
                out["selection"] = {key: c["selection"][key] for key in ("median_us", "min_us", "max_us")}
            return out

        entry = {
            "encoding": encoding, "m": m, "k": k, "rows": list(rows), "gflop": round(flops / 1e9, 3),
            "library_plan": chosen,
            "winner": public(winner),
            "library_us": library["selection"]["median_us"] if library else None,
            "winner_us": winner["selection"]["median_us"],
            "library_over_winner": round(library["selection"]["median_us"] / winner["selection"]["median_us"], 4)
            if library else None,
            "finalists": [public(c) for c in finalists],
            "candidates": [public(c) for c in sorted(candidates, key=lambda c: c["median_us"])],
        }
        report[name] = entry
        log("sweep", name, "library", (chosen["tile"], chosen["splits"]), entry["library_us"], "us; winner",
            (winner["tile"], winner["splits"]), entry["winner_us"], "us")
        for b in [*weights, x, *outs, workspace]:
            b.release()
    return report


GEMV_SWEEP_SHAPES = (("C2_q4k_gemv_m4_12288x4096", 4, 12288, 4096),
                     ("C2_q4k_gemv_m4_4096x12288", 4, 4096, 12288),
                     ("C2_q4k_gemv_m8_12288x4096", 8, 12288, 4096),
                     ("C2_q4k_gemv_m8_4096x12288", 8, 4096, 12288))


def gemv_plan_sweep(device, only=None):
    """Every multi-row plan of the Q4_K decode GEMV (kernel x launch fields) at C2's M=4 and M=8
    shapes, on rotated weight copies as the details cases run them, timed, then the three
    fastest re-timed before the winner is named, beside the plan the library picks (the
    protocol of ``plan_sweep``).  Each candidate's output is checked against the library
    plan's (rel-L2 <= 2e-3, no NaN) before it is timed."""
    from oracle import gguf_ref as R
    from tensor_amd.providers.hip import GEMV_FIELDS, GEMV_KERNELS
    from tests import gguf_cases as cases

    report = {}
    for name, m, n, k in GEMV_SWEEP_SHAPES:
        if only is not None and not name.startswith(only):
            continue
        chosen = device.gemv_plan("q4_k", m, k, n)
        copies = copies_for(weight_bytes("q4_k", n, k))
        weights = rotated(device, cases.weight(n, k, "q4_k", 1500 + m), copies)
        x = device.from_numpy(cases.activation(m, k, 1510 + m))
        out = device.empty((m, n), "float16")
        exe = device.load("gguf_gemv_variant", encoding="q4_k", out_dtype="float16")
        work = gemv_bytes("q4_k", m, n, k, 2)
        device.load("gguf_gemv", encoding="q4_k", out_dtype="float16").launch(x, weights[0], out)
        expected = out.to_numpy().astype(np.float32)
        candidates = []
        for kernel, fields in GEMV_FIELDS.items():
            for a, b in fields:
                try:
                    calls = [exe.bind(x, w, out, kernel=kernel, a=a, b=b) for w in weights]
                    device.fill_bytes(out, 0xFF)
                    calls[0].launch()
                except Exception as exc:  # the entry refuses plans that do not fit the shape
                    if getattr(exc, "code", None) == 2:
                        continue
                    raise
                got = out.to_numpy().astype(np.float32)
                ok = not np.isnan(got).any() and R.relative_l2(got, expected) <= 2e-3
                stats = time_launches(device, [calls[i % copies].launch for i in range(60)], per=60, replays=5)
                candidates.append({"kernel": kernel, "name": GEMV_KERNELS[kernel], "a": a, "b": b, "valid": bool(ok),
                                   "median_us": stats["median_us"], "calls": calls})
        finalists = sorted((c for c in candidates if c["valid"]), key=lambda c: c["median_us"])[:3]
        library = next(c for c in candidates if (c["kernel"], c["a"], c["b"]) == (chosen["kernel"], chosen["a"], chosen["b"]))
        for c in {id(c): c for c in [*finalists, library]}.values():
            c["selection"] = time_launches(device, [c["calls"][i % copies].launch for i in range(200)], per=200,
                                           replays=7)
        winner = min(finalists, key=lambda c: c["selection"]["median_us"])

        def public(c):
            out_ = {key: value for key, value in c.items() if key != "calls"}
            if "selection" in c:
                out_["selection"] = {key: c["selection"][key] for key in ("median_us", "min_us", "max_us")}
                out_["hbm_frac"] = round(work / c["selection"]["median_us"] * 1e-3 / HBM_PEAK_GBS, 4)
            return out_

        entry = {"m": m, "n": n, "k": k, "bytes": work, "copies": copies, "library_plan": chosen,
                 "winner": public(winner), "library_us": library["selection"]["median_us"],
                 "winner_us": winner["selection"]["median_us"],
                 "library_over_winner": round(library["selection"]["median_us"] / winner["selection"]["median_us"], 4),
                 "finalists": [public(c) for c in finalists],
                 "candidates": [public(c) for c in sorted(candidates, key=lambda c: c["median_us"])]}
        report[name] = entry
        log("sweep", name, "library", (chosen["name"], chosen["a"], chosen["b"]), entry["library_us"], "us; winner",
            (winner["name"], winner["a"], winner["b"]), entry["winner_us"], "us")
        for buffer in [*weights, x, out]:
            buffer.release()
    return report


# ------------------------------------------------------------------- main --

def main():
    global TIMING, WARM_SECONDS
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=300)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-details", action="store_true", help="headline only")
    parser.add_argument("--no-torch", action="store_true", help="skip the resident-dequantized torch.mm leg")
    parser.add_argument("--cpu-seconds", type=float, default=20.0)
    parser.add_argument("--calibrate", action="store_true",
                        help="first run 5 device copies of 256 MiB (a known-size copy kernel for PMC scaling)")
    parser.add_argument("--timing", choices=("graph", "eager"), default="graph",
                        help="replay each timed sequence from a captured HIP graph, or enqueue it eagerly")
    parser.add_argument("--only", metavar="PREFIX",
                        help="run only the details cases whose name starts with PREFIX (for profiling one kernel)")
    parser.add_argument("--eager-only", action="store_true",
                        help="stop after the eager warmup launches (for per-dispatch counter runs)")
    parser.add_argument("--warm-seconds", type=float, default=WARM_SECONDS,
                        help="untimed replay before each timed sequence (0: one replay, e.g. for counter runs)")
    parser.add_argument("--sweep", action="store_true",
                        help="time every tile and K split of the prefill GEMM at the BASELINE shapes and every "
                             "multi-row plan of the Q4_K decode GEMV at C2's M=4 / M=8 shapes, re-time the three "
                             "fastest, and print the winners beside the library's plans (one JSON line)")
    parser.add_argument("--torch-leg", action="store_true", help=argparse.SUPPRESS)
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        parser.error("steps must be >= 1 and warmup >= 0")
    TIMING = args.timing
    WARM_SECONDS = max(0.0, args.warm_seconds)
    if args.torch_leg:
        torch_leg()
        return 0

    sys.path.insert(0, ROOT)
    import tensor_amd as tx

    device = tx.Device(0, provider="hip")
    with device:
        log("device", device.info["name"], device.info["arch_features"], "CUs", device.info["compute_units"])
        if args.sweep:
            print(json.dumps({"plan_sweep": plan_sweep(device, args.only),
                              "gemv_plan_sweep": gemv_plan_sweep(device, args.only), "replays": REPLAYS,
                              "timing": "HIP graph replays, median; GEMM finalists re-timed over 7 replays of 60 "
                                        "launches, GEMV finalists over 7 replays of 200 launches on rotated weights"}))
            return 0
        if args.calibrate:
            source = device.zeros((256 << 20,), "uint8")
            target = device.empty((256 << 20,), "uint8")
            for _ in range(5):
                target.copy_from(source)
            device.synchronize()
            source.release()
            target.release()
            log("calibration: 5 device copies of", 256 << 20, "bytes")
        # ---- headline: C2 Q4_K GEMV M=1, one decode MLP per step: gate + up as one
        # grouped launch (they share x), then down
        per_step_weights = 2 * weight_bytes("q4_k", 12288, 4096) + weight_bytes("q4_k", 4096, 12288)
        copies = copies_for(per_step_weights)
        log("headline weights", per_step_weights, "B per step,", copies, "rotated copies")
        gate_up = GroupLinear(device, "q4_k", 1, [(12288, 4096), (12288, 4096)], "float16", copies, 1)
        down = Linear(device, "gguf_gemv", "q4_k", 1, 4096, 12288, "float16", copies, 5)
        mlp = [gate_up, down]
        step_bytes = gate_up.bytes + down.bytes
        for launch in rotated_launches(mlp, args.warmup):
            launch()
        device.synchronize()
        log("warmup done", args.warmup, "steps")
        if args.eager_only:
            for layer in mlp:
                layer.release()
            return 0
        headline = time_launches(device, rotated_launches(mlp, args.steps), per=args.steps)
        seconds = headline["median_us"] * 1e-6 * args.steps
        value = step_bytes * args.steps / seconds / 1e9
        log(f"headline {value:.1f} GB/s, {headline['median_us']:.2f} us/step "
            f"(min {headline['min_us']}, max {headline['max_us']})")

        # ---- roofline of the dominant kernel: the grouped gate + up GEMV, 2 x 12288 x 4096, M=1.
        # achieved / frac / avg_us are the committed rocprofv3 per-dispatch average of this kernel
        # (profiles/gemv_q4k_m1_qwen3_mlp.md); this run's own HIP-event timings sit beside them
        # under "live": the same 200 launches enqueued eagerly (host enqueue ~5 us per launch,
        # below the kernel's time, so the stream stays busy) and replayed from a captured graph.
        launches = 200
        sequence = [gate_up.calls[i % copies].launch for i in range(launches)]
        graph = time_launches(device, sequence, per=launches)
        TIMING, mode = "eager", TIMING
        eager = time_launches(device, sequence, per=launches)
        TIMING = mode
        figures = profile_figures()
        def live_figure(stats, how):
            return {"avg_us": stats["median_us"], "avg_us_min": stats["min_us"], "avg_us_max": stats["max_us"],
                    "achieved": round(gate_up.bytes / stats["median_us"] / 1e3, 1),
                    "frac": round(gate_up.bytes / stats["median_us"] / 1e3 / HBM_PEAK_GBS, 4),
                    "timing": f"HIP events on the launch stream around {launches} launches {how}, "
                              f"median of {REPLAYS} replays"}

        live = {"eager": live_figure(eager, "enqueued back to back"),
                "graph": live_figure(graph, "captured in one graph")}
        avg = figures.get("avg_us_per_launch", eager["median_us"])
        roofline = {
            "bound": "hbm",
            "achieved": round(gate_up.bytes / avg / 1e3, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gate_up.bytes / avg / 1e3 / HBM_PEAK_GBS, 4),
            "traffic": int(figures["traffic_bytes_per_launch"]) if "traffic_bytes_per_launch" in figures else None,
            "kernel": "gemv_q4k_m1<STEPS=1, WAVES=8, MATS=2> gate+up 2 x 12288x4096, M=1, fp16 out",
            "avg_us": avg,
            "timing": ("rocprofv3 --kernel-trace --stats per-dispatch average, profiles/gemv_q4k_m1_qwen3_mlp.md"
                       if "avg_us_per_launch" in figures else "live eager average (no committed profile)"),
            "algorithmic_bytes": gate_up.bytes,
            "live": live,
            "live_eager_vs_profiled": round(eager["median_us"] / avg, 4),
        }
        achieved = roofline["achieved"]
        log(f"roofline kernel: profiled {avg:.3f} us -> {achieved:.1f} GB/s; live eager {eager['median_us']:.3f} us, "
            f"graph {graph['median_us']:.3f} us")
        for layer in mlp:
            layer.release()

        details = {}
        if not args.no_details:
            details = run_details(device, args.only)
    if not args.no_details and not args.no_torch and args.only is None:
        details["torch_resident_dequantized_lower_bound"] = run_torch_leg()

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(seconds / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 x q4_k -> fp32 accumulate",
        "data": "synthetic: seeded N(0,0.02) weights quantized to Q4_K, N(0,1) fp16 activations",
        "config": {
            "workload": "C2 Q4_K decode GEMV, M=1, Qwen3-8B MLP step = gate 12288x4096 + up 12288x4096 "
                        "(one grouped launch sharing x) + down 4096x12288, fp16 out, weights rotated through "
                        f"{copies} copies ({copies * per_step_weights >> 20} MiB)",
            "M": 1,
            "hidden": 4096,
            "intermediate": 12288,
            "bytes_per_step": step_bytes,
            "timing": f"HIP graph of all K steps, HIP events on the launch stream, median of {REPLAYS} replays",
            "step_us": {k: v for k, v in headline.items()},
        },
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_seconds),
        "details": details,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
