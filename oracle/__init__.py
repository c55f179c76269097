"""CPU oracle for cuBlade's quantization numerics (TEST INFRASTRUCTURE ONLY).

This package wraps ``oracle/_build/libcbq_oracle.so`` (built from
``oracle/cbq_oracle.c`` by ``oracle/Makefile``) with numpy-facing helpers.
It is the checker the HIP kernels are compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; nothing under ``cublade_amd/`` does.

Array conventions: fp16 / bf16 tensors travel as ``np.uint16`` bit patterns,
FP8 E4M3 codes as ``np.uint8``, INT8 codes as ``np.int8``, scales as
``np.float32``. Dtype codes: 0 = fp32, 1 = fp16, 2 = bf16.

Each function's restated reference location is cited in ``cbq_oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
LIB_PATH = ROOT / "_build" / "libcbq_oracle.so"

F32, F16, BF16 = 0, 1, 2

_lib = None


def build(force: bool = False) -> Path:
    """Compile the C restatement with the committed Makefile."""
    if force or not LIB_PATH.exists():
        cmd = ["make", "-C", str(ROOT)]
        if force:
            subprocess.run(["make", "-C", str(ROOT), "clean"], check=True,
                           stdout=subprocess.DEVNULL)
        subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _declare(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def _declare(L: ctypes.CDLL) -> ctypes.CDLL:
    P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
    sig = {
        "cbo_f16_to_f32": (F, [ctypes.c_uint16]),
        "cbo_bf16_to_f32": (F, [ctypes.c_uint16]),
        "cbo_e4m3_to_f32": (F, [ctypes.c_uint8]),
        "cbo_f32_to_f16": (ctypes.c_uint16, [F]),
        "cbo_f32_to_bf16": (ctypes.c_uint16, [F]),
        "cbo_f32_to_e4m3_satfinite": (ctypes.c_uint8, [F]),
        "cbo_round_clamp_int8": (ctypes.c_int8, [F]),
        "cbo_load_f32": (None, [P, I32, I64, P]),
        "cbo_store_from_f32": (None, [P, I64, P, I32]),
        "cbo_cast_e4m3": (None, [P, I64, P]),
        "cbo_decode_e4m3": (None, [P, I64, P]),
        "cbo_cast_int8": (None, [P, I64, P]),
        "cbo_amax": (F, [P, I32, I64]),
        "cbo_inv_scale": (F, [F, F, F]),
        "cbo_scale_from_inv": (F, [F]),
        "cbo_quant_fp8_tensor": (I32, [P, I32, I64, F, P, P]),
        "cbo_quant_int8_tensor": (I32, [P, I32, I64, F, P, P]),
        "cbo_quant_int8_channel": (I32, [P, I32, I64, I64, I32, F, P, P]),
        "cbo_quant_int8_group": (I32, [P, I32, I64, I64, F, P, P]),
        "cbo_dequant_fp8_tensor": (I32, [P, P, I64, P, I32]),
        "cbo_dequant_int8_tensor": (I32, [P, P, I64, P, I32]),
        "cbo_dequant_int8_channel": (I32, [P, P, I64, I64, I32, P, I32]),
        "cbo_dequant_int8_group": (I32, [P, P, I64, I64, P, I32]),
        "cbo_mm_int8": (I32, [P, P, I32, I32, I64, I64, I64, P]),
        "cbo_mm_float": (I32, [P, P, I32, I32, I64, I64, I64, P]),
        "cbo_w8a16_linear": (I32, [P, I32, P, I64, P, P, P, P, I64, P,
                                   I64, I64, I64, P, I64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _fdtype_np(dtype_code: int):
    return np.float32 if dtype_code == F32 else np.uint16


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what}: invalid arguments (rc={rc})")


# ---------------------------------------------------------------------------
# element-wise conversions
# ---------------------------------------------------------------------------
def to_f32(x: np.ndarray, dtype_code: int) -> np.ndarray:
    x = _c(x, _fdtype_np(dtype_code))
    out = np.empty(x.shape, np.float32)
    lib().cbo_load_f32(_ptr(x), dtype_code, x.size, _ptr(out))
    return out


def from_f32(v: np.ndarray, dtype_code: int) -> np.ndarray:
    v = _c(v, np.float32)
    out = np.empty(v.shape, _fdtype_np(dtype_code))
    lib().cbo_store_from_f32(_ptr(v), v.size, _ptr(out), dtype_code)
    return out


def cast_e4m3(v: np.ndarray) -> np.ndarray:
    v = _c(v, np.float32)
    out = np.empty(v.shape, np.uint8)
    lib().cbo_cast_e4m3(_ptr(v), v.size, _ptr(out))
    return out


def decode_e4m3(q: np.ndarray) -> np.ndarray:
    q = _c(q, np.uint8)
    out = np.empty(q.shape, np.float32)
    lib().cbo_decode_e4m3(_ptr(q), q.size, _ptr(out))
    return out


def cast_int8(v: np.ndarray) -> np.ndarray:
    v = _c(v, np.float32)
    out = np.empty(v.shape, np.int8)
    lib().cbo_cast_int8(_ptr(v), v.size, _ptr(out))
    return out


def amax(x: np.ndarray, dtype_code: int) -> float:
    x = _c(x, _fdtype_np(dtype_code))
    return float(lib().cbo_amax(_ptr(x), dtype_code, x.size))


def inv_scale(amax_v: float, eps: float, qmax: float) -> np.float32:
    return np.float32(lib().cbo_inv_scale(amax_v, eps, qmax))


def scale_from_inv(inv: float) -> np.float32:
    return np.float32(lib().cbo_scale_from_inv(inv))


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------
def quant_fp8_tensor(x: np.ndarray, dtype_code: int, eps: float = 1e-12):
    """Returns (q uint8 codes shaped like x, scale np.float32)."""
    x = _c(x, _fdtype_np(dtype_code))
    q = np.empty(x.shape, np.uint8)
    s = np.zeros(1, np.float32)
    _check(lib().cbo_quant_fp8_tensor(_ptr(x), dtype_code, x.size, eps, _ptr(q), _ptr(s)),
           "quant_fp8_tensor")
    return q, s[0]


def quant_int8_tensor(x: np.ndarray, dtype_code: int, eps: float = 1e-12):
    x = _c(x, _fdtype_np(dtype_code))
    q = np.empty(x.shape, np.int8)
    s = np.zeros(1, np.float32)
    _check(lib().cbo_quant_int8_tensor(_ptr(x), dtype_code, x.size, eps, _ptr(q), _ptr(s)),
           "quant_int8_tensor")
    return q, s[0]


def quant_int8_channel(x: np.ndarray, dtype_code: int, axis: int = 0, eps: float = 1e-12):
    """x viewed as (rows, cols) = (x.shape[0], numel/rows); one scale per row
    (axis 0) or per column (axis 1)."""
    x = _c(x, _fdtype_np(dtype_code))
    rows = x.shape[0]
    cols = x.size // rows if rows else 0
    q = np.empty(x.shape, np.int8)
    s = np.zeros(rows if axis == 0 else cols, np.float32)
    _check(lib().cbo_quant_int8_channel(_ptr(x), dtype_code, rows, cols, axis, eps,
                                        _ptr(q), _ptr(s)), "quant_int8_channel")
    return q, s


def quant_int8_group(x: np.ndarray, dtype_code: int, group_size: int, eps: float = 1e-12):
    """x is (num_groups, group_size)-viewable; returns (q, scale[num_groups])."""
    x = _c(x, _fdtype_np(dtype_code))
    ng = x.size // group_size
    q = np.empty(x.shape, np.int8)
    s = np.zeros(ng, np.float32)
    _check(lib().cbo_quant_int8_group(_ptr(x), dtype_code, ng, group_size, eps,
                                      _ptr(q), _ptr(s)), "quant_int8_group")
    return q, s


# ---------------------------------------------------------------------------
# dequantization
# ---------------------------------------------------------------------------
def dequant_fp8_tensor(q: np.ndarray, scale: float, out_code: int) -> np.ndarray:
    q = _c(q, np.uint8)
    s = np.array([scale], np.float32)
    y = np.empty(q.shape, np.uint16)
    _check(lib().cbo_dequant_fp8_tensor(_ptr(q), _ptr(s), q.size, _ptr(y), out_code),
           "dequant_fp8_tensor")
    return y


def dequant_int8_tensor(q: np.ndarray, scale: float, out_code: int) -> np.ndarray:
    q = _c(q, np.int8)
    s = np.array([scale], np.float32)
    y = np.empty(q.shape, np.uint16)
    _check(lib().cbo_dequant_int8_tensor(_ptr(q), _ptr(s), q.size, _ptr(y), out_code),
           "dequant_int8_tensor")
    return y


def dequant_int8_channel(q: np.ndarray, scale: np.ndarray, out_code: int, axis: int = 0):
    q = _c(q, np.int8)
    s = _c(scale, np.float32)
    rows = q.shape[0]
    cols = q.size // rows if rows else 0
    y = np.empty(q.shape, np.uint16)
    _check(lib().cbo_dequant_int8_channel(_ptr(q), _ptr(s), rows, cols, axis, _ptr(y),
                                          out_code), "dequant_int8_channel")
    return y


def dequant_int8_group(q: np.ndarray, scale: np.ndarray, group_size: int, out_code: int):
    q = _c(q, np.int8)
    s = _c(scale, np.float32)
    ng = q.size // group_size
    y = np.empty(q.shape, np.uint16)
    _check(lib().cbo_dequant_int8_group(_ptr(q), _ptr(s), ng, group_size, _ptr(y), out_code),
           "dequant_int8_group")
    return y


# ---------------------------------------------------------------------------
# W8A16 linear
# ---------------------------------------------------------------------------
def w8a16_linear(x, act_code, wq, scales, bias=None, normal_cols=None,
                 outlier_cols=None, w_out=None, rows=None) -> np.ndarray:
    """Exact-accumulation W8A16 output (float32, shape [len(rows) or M, N]).

    x: [M, K] act bits; wq: int8 [N, Kn]; scales/bias: [N] act bits;
    normal_cols: int64 [Kn] or None; outlier_cols: int64 [n_out] or None;
    w_out: [N, n_out] act bits; rows: optional int64 row subset of x.
    """
    fd = _fdtype_np(act_code)
    x = _c(x, fd)
    M, K = x.shape
    wq = _c(wq, np.int8)
    N, Kn = wq.shape
    scales = _c(scales, fd)
    bias = None if bias is None else _c(bias, fd)
    nc = None if normal_cols is None else _c(normal_cols, np.int64)
    oc = None if outlier_cols is None else _c(outlier_cols, np.int64)
    n_out = 0 if oc is None else oc.size
    wo = None if w_out is None else _c(w_out, fd)
    r = None if rows is None else _c(rows, np.int64)
    R = M if r is None else r.size
    y = np.empty((R, N), np.float32)
    _check(lib().cbo_w8a16_linear(_ptr(x), act_code, _ptr(wq), Kn, _ptr(nc), _ptr(scales),
                                  _ptr(bias), _ptr(oc), n_out, _ptr(wo), M, N, K, _ptr(r),
                                  R, _ptr(y)), "w8a16_linear")
    return y


def mm_int8(a: np.ndarray, b: np.ndarray, b_nk: bool = False) -> np.ndarray:
    """C = a . b for int8 or uint8 operands, int32 accumulation wrapping modulo
    2^32 (wmma.cu:29-169 with int32 fragments). a: [M, K]; b: [K, N], or [N, K]
    when b_nk (b holds B^T)."""
    assert a.dtype == b.dtype and a.dtype in (np.int8, np.uint8)
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    M, K = a.shape
    N = b.shape[0] if b_nk else b.shape[1]
    assert (b.shape[1] if b_nk else b.shape[0]) == K
    c = np.empty((M, N), np.int32)
    _check(lib().cbo_mm_int8(_ptr(a), _ptr(b), int(a.dtype == np.uint8), int(b_nk), M, N, K,
                             _ptr(c)), "mm_int8")
    return c


def mm_float(a: np.ndarray, b: np.ndarray, dtype_code: int, b_nk: bool = False) -> np.ndarray:
    """C = a . b for fp16 / bf16 bit patterns (np.uint16), accumulated in
    double (wmma.cu:29-169 with fp32 fragments). Shapes as mm_int8."""
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    M, K = a.shape
    N = b.shape[0] if b_nk else b.shape[1]
    c = np.empty((M, N), np.float64)
    _check(lib().cbo_mm_float(_ptr(a), _ptr(b), dtype_code, int(b_nk), M, N, K, _ptr(c)),
           "mm_float")
    return c
