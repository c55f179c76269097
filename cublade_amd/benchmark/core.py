"""Timing helpers.

benchmark(): the reference's helper (benchmark/core.py:5-71: time a kernel
and a reference function, report TFLOP/s, gate with allclose) with device
timing: HIP events on the current stream, warm-up, median of repeats,
instead of the reference's unsynchronised perf_counter.

MallFlush: evicts the 256 MB Infinity Cache between timed launches with a
read-modify-write of a 512 MiB scratch buffer.
"""
from __future__ import annotations

import statistics
from typing import Callable, Optional

import torch

HBM_PEAK_BYTES_S = 8.0e12        # MI355X HBM3E
FP16_MFMA_PEAK_FLOP_S = 2.5e15   # MI355X dense fp16 / bf16 MFMA


class MallFlush:
    def __init__(self, device, nbytes: int = 512 << 20):
        self.buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=device)

    def __call__(self):
        self.buf.add_(1)


def time_op(fn: Callable[[], object], reps: int = 20, warmup: int = 3,
            flush: Optional[MallFlush] = None) -> list[float]:
    """Per-call device times in microseconds (HIP events on the current
    stream; the optional flush runs before each call, outside the events)."""
    for _ in range(warmup):
        if flush:
            flush()
        fn()
    stream = torch.cuda.current_stream()
    pairs = []
    for _ in range(reps):
        if flush:
            flush()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        pairs.append((a, b))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in pairs]


def benchmark(kernel_fn, ref_fn, *args, n_flop: Optional[float] = None, warmup: int = 3,
              reps: int = 20, atol: float = 1e-5, rtol: float = 1e-3):
    """Time kernel_fn(*args) (and ref_fn(*args) if given); returns a dict with
    median microseconds, TFLOP/s when n_flop is given, and the allclose gate."""
    out = {}
    k_us = statistics.median(time_op(lambda: kernel_fn(*args), reps, warmup))
    out["kernel_us"] = k_us
    if n_flop:
        out["kernel_tflops"] = n_flop / (k_us * 1e-6) / 1e12
    if ref_fn is not None:
        r_us = statistics.median(time_op(lambda: ref_fn(*args), reps, warmup))
        out["ref_us"] = r_us
        if n_flop:
            out["ref_tflops"] = n_flop / (r_us * 1e-6) / 1e12
        a, b = kernel_fn(*args), ref_fn(*args)
        out["allclose"] = bool(torch.allclose(a.float(), b.float(), atol=atol, rtol=rtol))
    return out
