"""CPU baseline for the benchmark: the oracle's CPU GEMM, timed.

TEST INFRASTRUCTURE ONLY (called from bench.py's cpu_baseline leg).

The GEMM the reference's callers run on the host is ``F.linear(x, W)``
(nanovllm/layers/linear.py:51) / ``torch.matmul`` (the reference's FP32
differential target); here it runs on PyTorch's CPU kernels in the input
dtype, multi-threaded.  The reference's own CPU timing precedent is a
single-thread float loop (cuda_kernels/gemm/src/gemm.cu:32-56); this
baseline is multi-threaded torch and is labelled so.
"""
from __future__ import annotations

import os
import platform
import time

import torch
import torch.nn.functional as F


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_cpu_gemm(a: torch.Tensor, b: torch.Tensor, b_layout_nk: bool, out_dtype: torch.dtype,
                  budget_s: float = 10.0, min_samples: int = 5, warmup: int = 2) -> dict:
    """Median seconds per GEMM on the host CPU, within a wall-clock budget.

    The sample is the full problem; at least `min_samples` timed calls are
    made unless one call alone exceeds the budget."""
    threads = torch.get_num_threads()

    def run():
        out = F.linear(a, b) if b_layout_nk else torch.matmul(a, b)
        return out if out.dtype == out_dtype else out.to(out_dtype)

    t_start = time.perf_counter()
    for _ in range(warmup):
        run()
        if time.perf_counter() - t_start > budget_s:
            break
    samples = []
    t0 = time.perf_counter()
    while len(samples) < min_samples or time.perf_counter() - t0 < budget_s / 4:
        s = time.perf_counter()
        run()
        samples.append(time.perf_counter() - s)
        if time.perf_counter() - t0 > budget_s:
            break
    samples.sort()
    return {
        "seconds": samples[len(samples) // 2],
        "samples": len(samples),
        "threads": threads,
        "cpu_count": os.cpu_count(),
        "cpu_model": cpu_model(),
    }
