"""Measurement subsystem: seeded BASELINE inputs (configs), device timing
with Infinity-Cache flushing (core), the per-config suite (suite) and
rocprofv3 result summaries (rocprof)."""
from .core import FP16_MFMA_PEAK_FLOP_S, HBM_PEAK_BYTES_S, MallFlush, benchmark, time_op

__all__ = ["benchmark", "time_op", "MallFlush", "HBM_PEAK_BYTES_S", "FP16_MFMA_PEAK_FLOP_S"]
