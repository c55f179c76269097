"""Helpers shared by the test modules: bit views, device upload, NaN-aware
bit comparisons."""
from __future__ import annotations

import numpy as np
import torch

import oracle

CODE_OF = {torch.float32: oracle.F32, torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}
DTYPE_OF = {v: k for k, v in CODE_OF.items()}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a tensor as numpy (uint16 for 16-bit floats, uint8
    for FP8, the native type otherwise)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy().copy()
    return t.numpy().copy()


def from_bits(a: np.ndarray, code: int, device="cpu") -> torch.Tensor:
    """Tensor of dtype DTYPE_OF[code] holding the bit pattern ``a``."""
    if code == oracle.F32:
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)
    t = torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16))
    return t.view(DTYPE_OF[code]).to(device)


def f16_nan_mask(b: np.ndarray, code: int) -> np.ndarray:
    b = np.asarray(b, np.uint16)
    if code == oracle.BF16:
        return (b & 0x7FFF) > 0x7F80
    return (b & 0x7FFF) > 0x7C00


def assert_bits_equal_16(got: np.ndarray, want: np.ndarray, code: int, what: str = ""):
    """16-bit float outputs equal bit for bit, except that any NaN matches any
    NaN (the NaN payload of a conversion is not part of the contract)."""
    got = np.asarray(got, np.uint16).reshape(-1)
    want = np.asarray(want, np.uint16).reshape(-1)
    assert got.shape == want.shape, what
    nan_w = f16_nan_mask(want, code)
    nan_g = f16_nan_mask(got, code)
    bad = (got != want) & ~(nan_w & nan_g)
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        raise AssertionError(f"{what}: {bad.sum()} of {got.size} differ; first at {i.tolist()}: "
                             f"got {[hex(v) for v in got[i]]} want {[hex(v) for v in want[i]]}")


def assert_fp8_equal(got: np.ndarray, want: np.ndarray, what: str = ""):
    got = np.asarray(got, np.uint8).reshape(-1)
    want = np.asarray(want, np.uint8).reshape(-1)
    assert got.shape == want.shape, what
    nan = ((want & 0x7F) == 0x7F) & ((got & 0x7F) == 0x7F)
    bad = (got != want) & ~nan
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        raise AssertionError(f"{what}: {bad.sum()} of {got.size} FP8 codes differ; first at "
                             f"{i.tolist()}: got {[hex(v) for v in got[i]]} "
                             f"want {[hex(v) for v in want[i]]}")


def assert_array_equal(got, want, what: str = ""):
    got = np.asarray(got).reshape(-1)
    want = np.asarray(want).reshape(-1)
    assert got.shape == want.shape, what
    bad = got != want
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        raise AssertionError(f"{what}: {bad.sum()} of {got.size} differ; first at {i.tolist()}: "
                             f"got {got[i].tolist()} want {want[i].tolist()}")


def assert_scales_equal(got: np.ndarray, want: np.ndarray, what: str = ""):
    assert_array_equal(np.asarray(got, np.float32).view(np.uint32),
                       np.asarray(want, np.float32).view(np.uint32), what + " scale bits")
