"""ctypes view of libcublade_quant.so (C ABI declared in include/cublade_quant.h).

Owns: the library handle and its function signatures, dtype codes, the HIP
stream of the current torch stream, and the per-(device, stream) workspace
whose first CBQ_WS_CTRL_BYTES bytes are a self-resetting control block.

There is no fallback: if the library cannot be built or loaded, every call
raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading

import torch

from ._loader import CSRC, load_hip_module

LIB_NAME = "cublade_quant"
SOURCES = [
    CSRC / "cbq_common.hip",
    CSRC / "cbq_quant.hip",
    CSRC / "cbq_dequant.hip",
    CSRC / "cbq_w8a16.hip",
    CSRC / "cbq_gemm.hip",
]

WS_CTRL_BYTES = 16384

F32, F16, BF16 = 0, 1, 2
I8, U8, I32 = 3, 4, 5
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
MM_DTYPE_CODE = {torch.int8: I8, torch.uint8: U8, torch.int32: I32, **DTYPE_CODE}
MM_B_KN, MM_B_NK = 0, 1

_P, _I64, _I32, _F, _SZ = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float,
                           ctypes.c_size_t)

# name -> (restype, argtypes); must match include/cublade_quant.h.
SIGNATURES = {
    "cbq_last_error": (ctypes.c_char_p, []),
    "cbq_abi_version": (_I32, []),
    "cbq_quant_tensor_ws_bytes": (_SZ, []),
    "cbq_quant_int8_channel_ws_bytes": (_SZ, [_I64, _I64, _I32]),
    "cbq_quant_fp8_tensor": (_I32, [_P, _I32, _I64, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_fp8_tensor_noalloc": (_I32, [_P, _I32, _I64, _F, _P, _P, _P]),
    "cbq_dequant_fp8_tensor": (_I32, [_P, _P, _I64, _P, _I32, _P]),
    "cbq_quant_int8_tensor": (_I32, [_P, _I32, _I64, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_channel": (_I32, [_P, _I32, _I64, _I64, _I32, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_group": (_I32, [_P, _I32, _I64, _I64, _F, _P, _P, _P]),
    "cbq_dequant_int8_tensor": (_I32, [_P, _P, _I64, _P, _I32, _P]),
    "cbq_dequant_int8_channel": (_I32, [_P, _P, _I64, _I64, _I32, _P, _I32, _P]),
    "cbq_dequant_int8_group": (_I32, [_P, _P, _I64, _I64, _P, _I32, _P]),
    "cbq_quant_int8_channel_nd_ws_bytes": (_SZ, [_I64, _I64, _I64]),
    "cbq_quant_int8_channel_nd": (_I32, [_P, _I32, _I64, _I64, _I64, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_group_nd": (_I32, [_P, _I32, _I64, _I64, _I64, _I64, _F, _P, _P, _P]),
    "cbq_dequant_int8_channel_nd": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _P]),
    "cbq_dequant_int8_group_nd": (_I32, [_P, _P, _I64, _I64, _I64, _I64, _P, _I32, _P]),
    "cbq_w8a16_ws_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "cbq_w8a16_linear": (_I32, [_P, _I32, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64,
                                _P, _SZ, _P, _P]),
    "cbq_mm_ws_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32]),
    "cbq_mm": (_I32, [_P, _P, _I32, _I32, _I64, _I64, _I64, _P, _I32, _P, _SZ, _P]),
}

_lib = None
_lib_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library (built on first use if no up-to-date build exists)."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                L = load_hip_module(LIB_NAME, SOURCES)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().cbq_last_error() or b""
        raise RuntimeError(f"{what}: {msg.decode(errors='replace')} (status {rc})")


def ptr(t: torch.Tensor | None):
    """Device address of t as an int (ctypes passes it as void*), or None."""
    return None if t is None else t.data_ptr()


# The current stream's raw hipStream_t as an int, without building a
# torch.cuda.Stream object (the public route costs ~3 us per call).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (0 is the null stream)."""
    idx = device_index(device)
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


_NO_SWITCH = contextlib.nullcontext()


def on_device(device: torch.device):
    """Context that makes `device` current for a launch; a no-op when it
    already is (entering torch.cuda.device costs ~2 us per call)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_SWITCH
    return torch.cuda.device(device)


_ws: dict[tuple[int, int], torch.Tensor] = {}
_ws_lock = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised workspace for (device, current stream), at least
    ``nbytes`` long. The library leaves its control block zeroed after every
    call, so the buffer is reused as-is; a larger request replaces it with a
    fresh zeroed one (allocated on the same stream, hence ordered)."""
    nbytes = max(int(nbytes), WS_CTRL_BYTES)
    key = (device_index(device), stream_handle(device))
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * (buf.numel() if buf is not None else 0), 1 << 12)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf
