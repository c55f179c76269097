"""Timing helpers.

benchmark(): the reference's helper (benchmark/core.py:5-71: time a kernel
and a reference function, report TFLOP/s, gate with allclose) with device
timing: HIP events on the current stream, warm-up, median of repeats,
instead of the reference's unsynchronised perf_counter.

MallFlush: evicts the 256 MB Infinity Cache (and the L2s) between timed
launches by sweeping a 512 MiB scratch buffer. The default sweep only reads,
so the caches are left holding clean lines and the timed kernel pays for no
other kernel's write-backs ("clean"); mode "dirty" writes the buffer instead,
leaving every cache line dirty (the worst case, as after a large producer).
Measured on MI355X, write-heavy kernels lose 15-20 points of HBM efficiency
after a dirty sweep; read-only streaming kernels do not change.
"""
from __future__ import annotations

import statistics
from typing import Callable, Optional

import torch

HBM_PEAK_BYTES_S = 8.0e12        # MI355X HBM3E
FP16_MFMA_PEAK_FLOP_S = 2.5e15   # MI355X dense fp16 / bf16 MFMA
I8_MFMA_PEAK_OP_S = 5.0e15       # MI355X dense int8 MFMA
FP32_PEAK_FLOP_S = 157.3e12      # MI355X fp32 (published)


class MallFlush:
    def __init__(self, device, nbytes: int = 512 << 20, mode: str = "clean"):
        if mode not in ("clean", "dirty"):
            raise ValueError(f"flush mode must be 'clean' or 'dirty', got {mode!r}")
        self.mode = mode
        # fp32 so that the reduction reads the buffer directly (an integer sum
        # would first widen the whole buffer into a temporary, i.e. write).
        self.buf = torch.zeros(nbytes // 4, dtype=torch.float32, device=device)
        self.sink = torch.zeros((), dtype=torch.float32, device=device)

    def __call__(self):
        if self.mode == "dirty":
            self.buf.add_(1.0)
        else:
            torch.sum(self.buf, dim=0, out=self.sink)


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
