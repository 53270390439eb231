"""A quick timing helper for one executable (the reference's ``tensor.runtime.bench``).

Three figures per call, each the median over ``iters`` samples:

* ``device``: the GPU time of one launch, from events recorded on the session stream
  around a batch of back-to-back launches (when the provider has events);
* ``launch_and_sync``: host wall time of one launch plus stream synchronization;
* ``host_enqueue``: host wall time of submitting one launch, without waiting.

The call is bound once (a BoundCall), so the figures exclude argument validation.
"""

from __future__ import annotations

import statistics
import time


def _median_and_min(samples):
    return statistics.median(samples), min(samples)


def bench(executable, buffers: tuple, *, warmup: int = 10, iters: int = 100, **bindings) -> dict:
    if type(warmup) is not int or warmup < 0 or type(iters) is not int or iters < 1:
        raise ValueError("warmup must be non-negative and iters must be positive")
    device = executable.device
    call = executable.bind(*buffers, **bindings)
    for _ in range(warmup):
        call.launch()
    device.synchronize()
    result = {"warmup": warmup, "iters": iters}

    synced = []
    for _ in range(iters):
        begin = time.perf_counter()
        call.launch()
        device.synchronize()
        synced.append(time.perf_counter() - begin)
    result["median_launch_and_sync_seconds"], result["min_launch_and_sync_seconds"] = _median_and_min(synced)

    enqueued = []
    for _ in range(iters):
        begin = time.perf_counter()
        call.launch()
        enqueued.append(time.perf_counter() - begin)
    device.synchronize()
    result["median_host_enqueue_seconds"] = statistics.median(enqueued)

    if "events" in getattr(device, "capabilities", ()):
        batch = 10
        per_launch = []
        for _ in range(iters):
            start = device.record_event(timing=True)
            for _ in range(batch):
                call.launch()
            stop = device.record_event(timing=True)
            stop.synchronize()
            per_launch.append(device.elapsed_ms(start, stop) * 1e-3 / batch)
            start.release()
            stop.release()
        result["median_device_seconds"], result["min_device_seconds"] = _median_and_min(per_launch)
    return result
