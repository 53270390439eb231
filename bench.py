"""Benchmark of the GGUF quantized-linear hot path on one MI355X.

Headline ("C2"): Q4_K decode GEMV at Qwen3-8B MLP
shapes, M = 1.  One *step* is one decode MLP's linears through the C ABI: gate
[12288 x 4096] and up [12288 x 4096] as one grouped launch (they share x), then
down [4096 x 12288].  ``value`` is the algorithmic bytes of all K steps
(packed weights + fp16 x + fp16 out) divided by the timed region.

Protocol (after benchmarks/kernels/showcase/benchmark.py:66-94): every launch
is bound once (allocation-free BoundCall), the K steps are captured into one
HIP graph, and the graph replay is timed with HIP events recorded on the
launch stream.  Weights rotate through distinct copies (>= 3 x 256 MiB per
rotation) so no launch finds its weights in the 256 MiB MALL.  Before the timed
replays every sequence is replayed, untimed, for WARM_SECONDS: an MI355X that
has idled through the host-side set-up of a case starts in deep sleep and needs
~30 ms of sustained load to reach its steady clocks (measured on the LM head:
123 us per launch over the first 100 launches, 93 us from the fourth hundred
on), so shorter warm-ups time the clock ramp instead of the kernel.

Also reported: ``roofline`` for the dominant kernel (the grouped gate + up
GEMV, 2 x 12288 x 4096; its HBM ``traffic`` is the per-launch figure measured
with rocprofv3 FETCH_SIZE / WRITE_SIZE and recorded in
profiles/gemv_q4k_m1_qwen3_mlp.md), ``cpu_baseline`` (the C restatement in
oracle/, invoked through its TensorKernelV1 entry exactly as the reference CPU
provider invokes images), and ``details`` for the other BASELINE
configurations (C2 M = 4/8 and the three-launch step, C3 LM head, C4 prefill
GEMM, C5 decoder-layer chain at M = 1 and M = 256).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FP16_PEAK_TFLOPS = 2516.6   # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20
ROTATION_BYTES = 3 * MALL_BYTES
METRIC = "Q4_K/Q6_K decode GEMV GB/s (% HBM peak); prefill dequant-GEMM TFLOP/s"
GEOMETRY = {"q4_0": (32, 18), "q8_0": (32, 34), "q4_k": (256, 144), "q6_k": (256, 210), "q4_1": (32, 20),
            "q5_0": (32, 22), "q5_1": (32, 24), "q2_k": (256, 84), "q3_k": (256, 110), "q5_k": (256, 176)}


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def weight_bytes(encoding, n, k):
    qk, block = GEOMETRY[encoding]
    return n * (k // qk) * block


def gemv_bytes(encoding, m, n, k, out_itemsize):
    return weight_bytes(encoding, n, k) + 2 * m * k + out_itemsize * m * n


class Linear:
    """One linear layer: R rotated weight copies, its input and output, bound calls."""

    def __init__(self, device, kernel, encoding, m, n, k, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        self.device, self.encoding, self.m, self.n, self.k = device, encoding, m, n, k
        self.out_dtype = out_dtype
        raw = cases.weight(n, k, encoding, seed)
        first = device.from_numpy(raw)
        self.weights = [first] + [device.empty(raw.shape, "uint8").copy_from(first) for _ in range(copies - 1)]
        self.x = x if x is not None else device.from_numpy(cases.activation(m, k, seed + 1))
        self.out = device.empty((m, n), out_dtype)
        self.exe = device.load(kernel, encoding=encoding, out_dtype=out_dtype)
        self.calls = [self.exe.bind(self.x, w, self.out) for w in self.weights]
        self.bytes = gemv_bytes(encoding, m, n, k, np.dtype(out_dtype).itemsize)
        self.flops = 2 * m * n * k

    def release(self):
        for b in self.weights + [self.out]:
            b.release()


class GroupLinear:
    """Matrices sharing one activation input, launched as one grouped GEMV call."""

    def __init__(self, device, encoding, m, shapes, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        k = shapes[0][1]
        assert all(sk == k for _, sk in shapes)
        self.device, self.encoding, self.m, self.k = device, encoding, m, k
        self.weights = []
        for i, (n, _) in enumerate(shapes):
            raw = cases.weight(n, k, encoding, seed + 2 * i)
            first = device.from_numpy(raw)
            self.weights.append([first] + [device.empty(raw.shape, "uint8").copy_from(first)
                                           for _ in range(copies - 1)])
        self.x = x if x is not None else device.from_numpy(cases.activation(m, k, seed + 1))
        self.outs = [device.empty((m, n), out_dtype) for n, _ in shapes]
        self.exe = device.load("gguf_gemv_group", encoding=encoding, out_dtype=out_dtype, count=len(shapes))
        self.calls = []
        for c in range(copies):
            args = [self.x]
            for ws, out in zip(self.weights, self.outs):
                args += [ws[c], out]
            self.calls.append(self.exe.bind(*args))
        itemsize = np.dtype(out_dtype).itemsize
        self.bytes = sum(weight_bytes(encoding, n, k) + itemsize * m * n for n, _ in shapes) + 2 * m * k
        self.flops = sum(2 * m * n * k for n, _ in shapes)

    def release(self):
        for ws in self.weights:
            for b in ws:
                b.release()
        for b in self.outs:
            b.release()


class SwigluLinear:
    """An MLP's gate and up matrices launched as one SwiGLU GEMV: out = silu(x Wg^T) * (x Wu^T)."""

    def __init__(self, device, encoding, m, n, k, out_dtype, copies, seed, x=None):
        from tests import gguf_cases as cases

        self.device, self.encoding, self.m, self.n, self.k = device, encoding, m, n, k
        self.weights = []
        for i in range(2):
            raw = cases.weight(n, k, encoding, seed + 2 * i)
            first = device.from_numpy(raw)
            self.weights.append([first] + [device.empty(raw.shape, "uint8").copy_from(first) for _ in range(copies - 1)])
        self.x = x if x is not None else device.from_numpy(cases.activation(m, k, seed + 1))
        self.out = device.empty((m, n), out_dtype)
        self.exe = device.load("gguf_gemv_swiglu", encoding=encoding, out_dtype=out_dtype)
        self.calls = [self.exe.bind(self.x, self.weights[0][c], self.weights[1][c], self.out) for c in range(copies)]
        self.bytes = 2 * weight_bytes(encoding, n, k) + 2 * m * k + np.dtype(out_dtype).itemsize * m * n
        self.flops = 4 * m * n * k

    def release(self):
        for ws in self.weights:
            for b in ws:
                b.release()
        self.out.release()


PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_q4k_m1_qwen3_mlp.md")


def measured_traffic():
    """HBM bytes per launch of the roofline kernel, from the committed rocprofv3 summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a 256 MiB copy); None if it is absent."""
    try:
        with open(PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copies_for(bytes_per_rotation_unit):
    return max(2, math.ceil(ROTATION_BYTES / bytes_per_rotation_unit))


TIMING = "graph"  # set from --timing in main()


def time_launches(device, launches, replays=3):
    """Median seconds of one pass over ``launches`` (callables), timed with HIP events on the
    launch stream: replayed from one captured HIP graph (``--timing graph``) or enqueued
    eagerly on the stream (``--timing eager``)."""
    if TIMING == "eager":
        return time_eager(device, launches, replays)
    return time_graph(device, launches, replays)


WARM_SECONDS = 0.1  # untimed replay before each timed sequence (steady clocks; module docstring)


def warm(device, run):
    """Call ``run`` (which enqueues GPU work) back to back until WARM_SECONDS have passed."""
    start = time.perf_counter()
    while True:
        run()
        device.synchronize()
        if time.perf_counter() - start >= WARM_SECONDS:
            return


def time_eager(device, launches, replays=3):
    warm(device, lambda: [launch() for launch in launches])
    samples = []
    for _ in range(replays):
        start = device.record_event(timing=True)
        for launch in launches:
            launch()
        stop = device.record_event(timing=True)
        stop.synchronize()
        samples.append(device.elapsed_ms(start, stop) * 1e-3)
        start.release()
        stop.release()
    return statistics.median(samples)


def time_graph(device, launches, replays=3):
    """Capture ``launches`` (callables) into one graph; return the median seconds of one replay."""
    graph = device.graph(lambda: [launch() for launch in launches])
    try:
        warm(device, graph.replay)
        samples = []
        for _ in range(replays):
            start = device.record_event(timing=True)
            graph.replay()
            stop = device.record_event(timing=True)
            stop.synchronize()
            samples.append(device.elapsed_ms(start, stop) * 1e-3)
            start.release()
            stop.release()
        return statistics.median(samples)
    finally:
        graph.close()


def rotated_launches(linears, steps):
    """``steps`` passes over the linears, each pass using the next weight copy."""
    out = []
    for step in range(steps):
        for layer in linears:
            out.append(layer.calls[step % len(layer.calls)].launch)
    return out


# ------------------------------------------------------------ CPU baseline --

def cpu_baseline(budget_s=10.0):
    """Time the oracle's TensorKernelV1 CPU entry on the headline step."""
    import ctypes as c

    from oracle import gguf_ref
    from tensor_amd.runtime import abi
    from tests import gguf_cases as cases

    if not gguf_ref.LIBRARY.exists():
        gguf_ref.build()
    oracle = gguf_ref.c_oracle()
    cores = min(16, len(os.sched_getaffinity(0)))
    layers = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
    copies = 4  # 340 MB of distinct weights per rotation (beyond the host LLC)
    data = []
    for i, (_, n, k) in enumerate(layers):
        first = cases.weight(n, k, "q4_k", 1000 + i)
        raws = [first] + [first.copy() for _ in range(copies - 1)]
        x = cases.activation(1, k, 2000 + i)
        out = np.empty((1, n), np.float16)
        data.append((raws, x, out, n, k))

    def call_for(x, raw, out):
        keep = []
        args = (abi.Argument * 4)()
        for j, (arr, dtype) in enumerate(((x, 10), (raw, 3), (out, 10))):
            shape = (c.c_int64 * 2)(*arr.shape)
            strides = (c.c_int64 * 2)(arr.strides[0], arr.strides[1])
            keep += [shape, strides]
            args[j].kind, args[j].dtype = 1, dtype
            args[j].buffer = abi.BufferDescriptor(arr.ctypes.data, arr.nbytes, shape, strides, 2, dtype, 1, 0)
        args[3].kind, args[3].dtype, args[3].scalar = 2, 7, 12
        call = abi.CallDescriptor(1, 72, args, 4, 0, (c.c_uint32 * 3)(1, 1, 1), (c.c_uint32 * 3)(1, 1, 1), 0,
                                  abi.StreamDescriptor(1, 0, 0))
        return call, keep, args

    calls = [[call_for(x, raw, out) for raw in raws] for raws, x, out, _, _ in data]
    entry = oracle.entry
    entry.argtypes = [c.POINTER(abi.CallDescriptor), c.POINTER(abi.ErrorDescriptor)]
    entry.restype = c.c_int32
    step_bytes = sum(gemv_bytes("q4_k", 1, n, k, 2) for _, _, _, n, k in data)

    def measure(threads, seconds):
        oracle.set_threads(threads)
        error = abi.ErrorDescriptor()
        samples, step, begin = [], 0, time.perf_counter()
        while time.perf_counter() - begin < seconds or len(samples) < 3:
            t0 = time.perf_counter()
            for layer in calls:
                status = entry(c.byref(layer[step % copies][0]), c.byref(error))
                if status:
                    raise RuntimeError(error.message.decode())
            samples.append(time.perf_counter() - t0)
            step += 1
        return statistics.median(samples), len(samples)

    multi, n_multi = measure(cores, budget_s * 0.75)
    single, n_single = measure(1, budget_s * 0.25)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(step_bytes / multi / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n_multi} steps of the headline step (Q4_K GEMV M=1 gate+up+down, {step_bytes} B/step), "
                  f"median {multi * 1e3:.2f} ms/step on {cores} threads; weights rotated over {copies} copies",
        "single_thread_gbs": round(step_bytes / single / 1e9, 3),
        "single_thread_ms_per_step": round(single * 1e3, 3),
        "cpu_model": model,
    }


# ------------------------------------------------------------------- main --

def main():
    global TIMING, WARM_SECONDS
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=300)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-details", action="store_true", help="headline only")
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
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
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        parser.error("steps must be >= 1 and warmup >= 0")
    TIMING = args.timing
    WARM_SECONDS = max(0.0, args.warm_seconds)

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import tensor_amd as tx

    device = tx.Device(0, provider="hip")
    with device:
        log("device", device.info["name"], device.info["arch_features"], "CUs", device.info["compute_units"])
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
        step_bytes = sum(layer.bytes for layer in mlp)
        for launch in rotated_launches(mlp, args.warmup):
            launch()
        device.synchronize()
        log("warmup done", args.warmup, "steps")
        if args.eager_only:
            for layer in mlp:
                layer.release()
            return 0
        seconds = time_launches(device, rotated_launches(mlp, args.steps), replays=3)
        value = step_bytes * args.steps / seconds / 1e9
        log(f"headline {value:.1f} GB/s, {seconds / args.steps * 1e6:.2f} us/step")

        # ---- roofline of the dominant kernel: the grouped gate + up GEMV, 2 x 12288 x 4096, M=1
        launches = 200
        kernel_s = time_launches(device, [gate_up.calls[i % copies].launch for i in range(launches)]) / launches
        achieved = gate_up.bytes / kernel_s / 1e9
        roofline = {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "kernel": "gemv_q4k_m1<STEPS=1, WAVES=8, MATS=2> gate+up 2 x 12288x4096, M=1, fp16 out",
            "avg_us": round(kernel_s * 1e6, 3),
            "algorithmic_bytes": gate_up.bytes,
        }
        log(f"roofline kernel {kernel_s * 1e6:.2f} us -> {achieved:.1f} GB/s")

        details = {}
        if not args.no_details:
            details = run_details(device, gate_up.x, log, args.only)
        for layer in mlp:
            layer.release()

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
            "timing": "HIP graph of all K steps, HIP events on the launch stream",
        },
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_seconds),
        "details": details,
    }
    print(json.dumps(result))
    return 0


def three_launch_step(device, x4096, log, details):
    """The headline step as three single-matrix launches (gate, up, down)."""
    copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096) + weight_bytes("q4_k", 4096, 12288))
    mlp = [Linear(device, "gguf_gemv", "q4_k", 1, 12288, 4096, "float16", copies, 1, x=x4096),
           Linear(device, "gguf_gemv", "q4_k", 1, 12288, 4096, "float16", copies, 3, x=x4096),
           Linear(device, "gguf_gemv", "q4_k", 1, 4096, 12288, "float16", copies, 5)]
    steps = 50
    seconds = time_launches(device, rotated_launches(mlp, steps)) / steps
    step_bytes = sum(layer.bytes for layer in mlp)
    details["C2_step_m1_three_launches"] = {"us": round(seconds * 1e6, 3),
                                            "GB/s": round(step_bytes / seconds / 1e9, 1),
                                            "hbm_frac": round(step_bytes / seconds / 1e9 / HBM_PEAK_GBS, 4)}
    log("C2_step_m1_three_launches", details["C2_step_m1_three_launches"])
    for layer in mlp:
        layer.release()


def run_details(device, x4096, log, only=None):
    """Per-config figures for the other BASELINE configurations (those whose name starts with
    ``only``, when given)."""
    details = {}

    def wanted(name):
        return only is None or name.startswith(only)

    def gemv_case(name, encoding, m, n, k, out_dtype, launches=60):
        if not wanted(name):
            return
        copies = copies_for(weight_bytes(encoding, n, k))
        layer = Linear(device, "gguf_gemv", encoding, m, n, k, out_dtype, copies, 7 + m)
        seconds = time_launches(device, [layer.calls[i % copies].launch for i in range(launches)]) / launches
        gbs = layer.bytes / seconds / 1e9
        details[name] = {"us": round(seconds * 1e6, 3), "GB/s": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
        log(name, details[name])
        layer.release()

    # the headline step as three single-matrix launches (gate, up, down)
    if wanted("C2_step_m1_three_launches"):
        three_launch_step(device, x4096, log, details)

    # the MLP as a decode step runs it: gate + up with the SwiGLU epilogue in one launch, then
    # down on its output (the headline step leaves the SwiGLU between them out)
    if wanted("C2_q4k_gemv_swiglu_m1_12288x4096") or wanted("C2_step_m1_swiglu"):
        copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096) + weight_bytes("q4_k", 4096, 12288))
        fused = SwigluLinear(device, "q4_k", 1, 12288, 4096, "float16", copies, 60, x=x4096)
        launches = 60
        seconds = time_launches(device, [fused.calls[i % copies].launch for i in range(launches)]) / launches
        gbs = fused.bytes / seconds / 1e9
        details["C2_q4k_gemv_swiglu_m1_12288x4096"] = {"us": round(seconds * 1e6, 3), "GB/s": round(gbs, 1),
                                                       "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
        log("C2_q4k_gemv_swiglu_m1_12288x4096", details["C2_q4k_gemv_swiglu_m1_12288x4096"])
        down = Linear(device, "gguf_gemv", "q4_k", 1, 4096, 12288, "float16", copies, 64, x=fused.out)
        steps = 50
        seconds = time_launches(device, rotated_launches([fused, down], steps)) / steps
        step_bytes = fused.bytes + down.bytes
        details["C2_step_m1_swiglu"] = {"us": round(seconds * 1e6, 3), "GB/s": round(step_bytes / seconds / 1e9, 1),
                                        "hbm_frac": round(step_bytes / seconds / 1e9 / HBM_PEAK_GBS, 4),
                                        "launches": 2}
        log("C2_step_m1_swiglu", details["C2_step_m1_swiglu"])
        down.release()
        fused.release()

    # C1's shape (the reference runs it on its CPU provider) on the GPU
    gemv_case("C1_q8_0_gemv_m1_4096x4096", "q8_0", 1, 4096, 4096, "float16")
    # C5's Q6_K down projection on its own
    gemv_case("C5_q6k_gemv_m1_4096x12288", "q6_k", 1, 4096, 12288, "float16")
    # gate + up as one grouped launch at M = 4 and 8
    for m in (4, 8):
        name = f"C2_q4k_gemv_group_m{m}_2x12288x4096"
        if wanted(name):
            copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096))
            group = GroupLinear(device, "q4_k", m, [(12288, 4096), (12288, 4096)], "float16", copies, 70 + m)
            seconds = time_launches(device, [group.calls[i % copies].launch for i in range(60)]) / 60
            gbs = group.bytes / seconds / 1e9
            details[name] = {"us": round(seconds * 1e6, 3), "GB/s": round(gbs, 1),
                             "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
            log(name, details[name])
            group.release()
    # the SwiGLU pair at M = 4 and 8
    for m in (4, 8):
        name = f"C2_q4k_gemv_swiglu_m{m}_12288x4096"
        if wanted(name):
            copies = copies_for(2 * weight_bytes("q4_k", 12288, 4096))
            pair = SwigluLinear(device, "q4_k", m, 12288, 4096, "float16", copies, 66 + m)
            seconds = time_launches(device, [pair.calls[i % copies].launch for i in range(60)]) / 60
            gbs = pair.bytes / seconds / 1e9
            details[name] = {"us": round(seconds * 1e6, 3), "GB/s": round(gbs, 1),
                             "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
            log(name, details[name])
            pair.release()
    for m in (1, 4, 8):
        gemv_case(f"C2_q4k_gemv_m{m}_12288x4096", "q4_k", m, 12288, 4096, "float16")
        gemv_case(f"C2_q4k_gemv_m{m}_4096x12288", "q4_k", m, 4096, 12288, "float16")
    gemv_case("C3_q6k_lm_head_m1_151936x4096_fp32", "q6_k", 1, 151936, 4096, "float32", launches=20)
    # every other encoding at the C2 gate shape, M = 1 (Q6_K, Q8_0 and Q4_0 on their own kernels,
    # the rest on the generic per-element decoder)
    for encoding in ("q6_k", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q5_k"):
        gemv_case(f"enc_{encoding}_gemv_m1_12288x4096", encoding, 1, 12288, 4096, "float16")

    def gemm_case(name, encoding, m, n, k, launches=10):
        if not wanted(name):
            return
        layer = Linear(device, "gguf_gemm", encoding, m, n, k, "float16", 2, 9)
        seconds = time_launches(device, [layer.calls[i % 2].launch for i in range(launches)]) / launches
        tflops = layer.flops / seconds / 1e12
        details[name] = {"us": round(seconds * 1e6, 2), "TFLOP/s": round(tflops, 2),
                         "mfma_frac": round(tflops / FP16_PEAK_TFLOPS, 4)}
        log(name, details[name])
        layer.release()

    gemm_case("C4_q4k_gemm_m512_12288x4096", "q4_k", 512, 12288, 4096)
    for encoding in ("q5_k", "q8_0", "q4_0"):
        gemm_case(f"enc_{encoding}_gemm_m512_12288x4096", encoding, 512, 12288, 4096)
    gemm_case("C4_q4k_gemm_m2048_12288x4096", "q4_k", 2048, 12288, 4096, launches=4)

    # C5: q, k, v, o, gate, up (Q4_K) and down (Q6_K) chained on one stream
    shapes = [("q", "q4_k", 4096, 4096), ("k", "q4_k", 1024, 4096), ("v", "q4_k", 1024, 4096),
              ("o", "q4_k", 4096, 4096), ("gate", "q4_k", 12288, 4096), ("up", "q4_k", 12288, 4096),
              ("down", "q6_k", 4096, 12288)]
    layer_weights = sum(weight_bytes(e, n, k) for _, e, n, k in shapes)
    for m, kernel in ((1, "gguf_gemv"), (256, "gguf_gemm")):
        if not wanted(f"C5_layer_m{m}"):
            continue
        copies = copies_for(layer_weights) if m == 1 else 2
        layers = [Linear(device, kernel, e, m, n, k, "float16", copies, 20 + i) for i, (_, e, n, k) in enumerate(shapes)]
        steps = 20 if m == 1 else 4
        seconds = time_launches(device, rotated_launches(layers, steps)) / steps
        total_bytes = sum(layer.bytes for layer in layers)
        total_flops = sum(layer.flops for layer in layers)
        details[f"C5_layer_m{m}"] = {
            "us": round(seconds * 1e6, 2),
            "GB/s": round(total_bytes / seconds / 1e9, 1),
            "TFLOP/s": round(total_flops / seconds / 1e12, 2),
        }
        log(f"C5_layer_m{m}", details[f"C5_layer_m{m}"])
        for layer in layers:
            layer.release()
    # C5 at M=1 the way a decode step runs it: q + k + v grouped, o, gate + up grouped, down
    if not wanted("C5_layer_m1_grouped"):
        return details
    copies = copies_for(layer_weights)
    x = device.from_numpy(np.zeros((1, 4096), np.float16) + np.float16(0.5))
    layers = [GroupLinear(device, "q4_k", 1, [(4096, 4096), (1024, 4096), (1024, 4096)], "float16", copies, 40, x=x),
              Linear(device, "gguf_gemv", "q4_k", 1, 4096, 4096, "float16", copies, 46, x=x),
              GroupLinear(device, "q4_k", 1, [(12288, 4096), (12288, 4096)], "float16", copies, 48, x=x),
              Linear(device, "gguf_gemv", "q6_k", 1, 4096, 12288, "float16", copies, 52)]
    steps = 20
    seconds = time_launches(device, rotated_launches(layers, steps)) / steps
    total_bytes = sum(layer.bytes for layer in layers)
    details["C5_layer_m1_grouped"] = {"us": round(seconds * 1e6, 2), "GB/s": round(total_bytes / seconds / 1e9, 1),
                                      "launches": 4}
    log("C5_layer_m1_grouped", details["C5_layer_m1_grouped"])
    for layer in layers:
        layer.release()
    x.release()
    return details


if __name__ == "__main__":
    sys.exit(main())
