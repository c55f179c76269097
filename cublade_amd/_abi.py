"""ctypes view of libcublade_quant.so (C ABI declared in include/cublade_quant.h).

Owns: the library handle and its function signatures, dtype codes, the HIP
stream of the current torch stream, and the per-(device, stream) workspace
whose first CBQ_WS_CTRL_BYTES bytes are the library's control block (zero
when created; the library keeps state there between calls).

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
# The library's ABI major version these signatures match (cbq_abi_version() // 100).
ABI_MAJOR = 2

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
    "cbq_tensor_quant_status": (_I32, [_P, _P, ctypes.POINTER(ctypes.c_int)]),
    "cbq_tensor_quant_status_clear": (_I32, [_P, _P]),
    "cbq_set_tensor_spin_limit": (ctypes.c_uint32, [ctypes.c_uint32]),
    "cbq_dequant_fp8_tensor": (_I32, [_P, _P, _I64, _P, _I32, _P]),
    "cbq_quant_int8_tensor": (_I32, [_P, _I32, _I64, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_channel": (_I32, [_P, _I32, _I64, _I64, _I32, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_group": (_I32, [_P, _I32, _I64, _I64, _F, _P, _P, _P]),
    "cbq_dequant_int8_tensor": (_I32, [_P, _P, _I64, _P, _I32, _P]),
    "cbq_dequant_int8_channel": (_I32, [_P, _P, _I64, _I64, _I32, _P, _I32, _P]),
    "cbq_dequant_int8_group": (_I32, [_P, _P, _I64, _I64, _P, _I32, _P]),
    "cbq_quant_int8_channel_nd_ws_bytes": (_SZ, [_I64, _I64, _I64]),
    "cbq_quant_int8_channel_nd": (_I32, [_P, _I32, _I64, _I64, _I64, _F, _P, _SZ, _P, _P, _P]),
    "cbq_quant_int8_group_nd_ws_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "cbq_quant_int8_group_nd": (_I32, [_P, _I32, _I64, _I64, _I64, _I64, _F, _P, _SZ, _P, _P,
                                       _P]),
    "cbq_dequant_int8_channel_nd": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _P]),
    "cbq_dequant_int8_group_nd_ws_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "cbq_dequant_int8_group_nd": (_I32, [_P, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P, _I32,
                                         _P]),
    "cbq_w8a16_ws_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
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
                L.cbq_abi_version.restype = _I32
                L.cbq_abi_version.argtypes = []
                ver = L.cbq_abi_version()
                if ver // 100 != ABI_MAJOR:
                    raise RuntimeError(
                        f"cublade: {LIB_NAME} has ABI version {ver}, these bindings need major "
                        f"version {ABI_MAJOR} (rebuild the library)")
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
# Workspaces replaced by a larger one. They are never freed: a HIP graph
# captured on that stream may hold their address (the per-tensor control
# block, split-K partials) and replays would otherwise write into memory
# the caching allocator has handed to another tensor.
_ws_retired: list[torch.Tensor] = []
_ws_lock = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Workspace for (device, current stream), at least ``nbytes`` long,
    zero-filled when created. The library keeps state in its control block
    between calls (the one-launch per-tensor quant's call count and slots),
    so the buffer is reused as-is. A larger request replaces it with a fresh
    zero-filled one (allocated on the same stream, hence ordered); the old
    one is kept alive for graphs captured with it. Growing during a graph
    capture raises: run one call of each captured shape on the capture
    stream first."""
    nbytes = max(int(nbytes), WS_CTRL_BYTES)
    key = (device_index(device), stream_handle(device))
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"cublade: the workspace of the capture stream must grow to {nbytes} bytes "
                    f"during graph capture; run one call of every captured shape on that stream "
                    f"before capturing")
            size = max(nbytes, 2 * (buf.numel() if buf is not None else 0), 1 << 12)
            new = torch.zeros(size, dtype=torch.uint8, device=device)
            if buf is not None:
                _ws_retired.append(buf)
            _ws[key] = new
            buf = new
        return buf


def _tensor_ws(device: torch.device):
    key = (device_index(device), stream_handle(device))
    with _ws_lock:
        return _ws.get(key)


def tensor_quant_status(device: torch.device, noalloc: bool = False) -> int:
    """The sticky status word of the one-launch per-tensor quant: of the
    current stream's workspace, or with ``noalloc`` of the static array that
    cbq_quant_fp8_tensor_noalloc uses on ``device``. 0: no exchange timed out
    since the word was last cleared; 1: one did (that call's scale is NaN
    unless every code it wrote is exact; later calls are exact again).
    Synchronises the current stream."""
    buf = None if noalloc else _tensor_ws(device)
    if buf is None and not noalloc:
        return 0
    st = ctypes.c_int(0)
    with on_device(device):
        check(lib().cbq_tensor_quant_status(None if noalloc else buf.data_ptr(),
                                            stream_handle(device), ctypes.byref(st)),
              "cbq_tensor_quant_status")
    return st.value


def clear_tensor_quant_status(device: torch.device, noalloc: bool = False) -> None:
    """Clears that status word, in stream order (no synchronisation)."""
    buf = None if noalloc else _tensor_ws(device)
    if buf is None and not noalloc:
        return
    with on_device(device):
        check(lib().cbq_tensor_quant_status_clear(None if noalloc else buf.data_ptr(),
                                                  stream_handle(device)),
              "cbq_tensor_quant_status_clear")


def set_tensor_spin_limit(polls: int) -> int:
    """Polls before a per-tensor quant's workgroups give up waiting for each
    other (cbq_set_tensor_spin_limit); returns the previous value."""
    return int(lib().cbq_set_tensor_spin_limit(int(polls)))
