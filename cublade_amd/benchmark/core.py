"""Timing helpers.

benchmark(): the reference's helper (benchmark/core.py:5-71) with the same
signature, printed table and returned dict (time a kernel and a reference
function, GFLOPS from the required n_flop, max abs error, allclose gate), but
timed on the device: a function whose output lives on the GPU is timed with
HIP events on the current stream (median of `reps` calls after `warmup`),
instead of the reference's single unsynchronised perf_counter interval, which
measures only the launch; a function with a CPU output is timed with
perf_counter (median of `reps`).

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
import time
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


def _median_ms(fn, args, reps: int) -> float:
    """Median milliseconds of fn(*args): HIP events on the current stream if
    its output is a GPU tensor, perf_counter otherwise."""
    out = fn(*args)
    if isinstance(out, torch.Tensor) and out.is_cuda:
        return statistics.median(time_op(lambda: fn(*args), reps, 0)) / 1e3
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn(*args)
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def benchmark(kernel_fn, ref_fn, *args, n_flop: int, warmup: int = 1, atol: float = 1e-5,
              rtol: float = 1e-3, reps: int = 20):
    """Compare a custom kernel against a reference implementation (the
    reference's contract, benchmark/core.py:5-71).

    Prints the reference's table (function, time in ms, GFLOPS, max abs error,
    PASS/FAIL/REF) and returns
        {"kernel":    {"time_ms", "gflops", "max_err", "passed", "output"},
         "reference": {"time_ms", "gflops", "output"}}
    Times are medians of `reps` device-timed calls after `warmup` calls of
    each (see the module docstring)."""
    for _ in range(warmup):
        kernel_fn(*args)
        ref_fn(*args)
    ms_ref = _median_ms(ref_fn, args, reps)
    ms_k = _median_ms(kernel_fn, args, reps)
    gflops_ref = n_flop / (ms_ref * 1e6)
    gflops_k = n_flop / (ms_k * 1e6)
    out_ref = ref_fn(*args)
    out_k = kernel_fn(*args)
    if isinstance(out_ref, torch.Tensor) and isinstance(out_k, torch.Tensor) and \
            out_ref.device != out_k.device:
        out_ref_cmp = out_ref.to(out_k.device)
    else:
        out_ref_cmp = out_ref
    max_err = (out_k - out_ref_cmp).abs().max().item()
    passed = torch.allclose(out_k, out_ref_cmp, rtol=rtol, atol=atol)

    header = f"{'Function':<20} {'Time (ms)':>10} {'GFLOPS':>10} {'max_err':>12} {'Status':>8}"
    print(header)
    print("-" * len(header))
    print(f"{getattr(ref_fn, '__name__', 'reference'):<20} {ms_ref:10.4f} {gflops_ref:10.1f} "
          f"{'-':>12} {'REF':>8}")
    print(f"{getattr(kernel_fn, '__name__', 'kernel'):<20} {ms_k:10.4f} {gflops_k:10.1f} "
          f"{max_err:12.2e} {'PASS' if passed else 'FAIL':>8}")
    return {
        "kernel": {"time_ms": ms_k, "gflops": gflops_k, "max_err": max_err, "passed": passed,
                   "output": out_k},
        "reference": {"time_ms": ms_ref, "gflops": gflops_ref, "output": out_ref},
    }
