"""dequantize_tensor (reference: quantization/dequantizers.py:18-75).

Output dtype is ``qt.original_dtype`` (fp16 / bf16 only, as in the
reference). Channel mode accepts any axis and group mode any axis, in place
(see quantizers).
"""
from __future__ import annotations

import torch

from .quantizers import channel_kernel_axis
from .tensor import QuantizedTensor
from cublade_amd.bindings.hip.dequantize_fp8 import (
    dequantize_per_tensor_fp8 as _hip_dequant_fp8_tensor,
)
from cublade_amd.bindings.hip.dequantize_int8 import (
    dequantize_per_tensor_int8 as _hip_dequant_int8_tensor,
    dequantize_per_channel_int8 as _hip_dequant_int8_channel,
    dequantize_per_group_int8 as _hip_dequant_int8_group,
    dequantize_per_channel_int8_nd as _hip_dequant_int8_channel_nd,
    dequantize_per_group_int8_nd as _hip_dequant_int8_group_nd,
)

_INT8_DTYPES = (torch.int8,)
_FP8_DTYPES = (torch.float8_e4m3fn,)


def _require_cuda_dequant_input(q: torch.Tensor, out_dtype: torch.dtype, *, what: str) -> None:
    """Checks of dequantizers.py:18-32."""
    if not q.is_cuda:
        raise ValueError(f"{what}: tensor must be on CUDA, got device={q.device}")
    if not q.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if q.dtype not in _INT8_DTYPES + _FP8_DTYPES:
        raise ValueError(
            f"{what}: q.dtype must be torch.int8 or torch.float8_e4m3fn, got {q.dtype}"
        )
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"{what}: out_dtype must be float16 or bfloat16, got {out_dtype}")


def dequantize_tensor(qt: QuantizedTensor) -> torch.Tensor:
    """Dequantize a QuantizedTensor: y = (float(q) * scale).to(original_dtype)."""
    _require_cuda_dequant_input(qt.data, qt.original_dtype, what="dequantize_tensor")

    if qt.dtype == torch.float8_e4m3fn:
        if qt.mode != "tensor":
            raise NotImplementedError("FP8 dequant only supports mode='tensor'")
        return _hip_dequant_fp8_tensor(qt.data, qt.scale, qt.original_dtype)

    if qt.dtype == torch.int8:
        if qt.mode == "tensor":
            return _hip_dequant_int8_tensor(qt.data, qt.scale, qt.original_dtype)
        if qt.mode == "channel":
            axis = channel_kernel_axis(qt.data.dim(), qt.axis)
            if axis == 0:
                return _hip_dequant_int8_channel(qt.data, qt.scale, qt.original_dtype)
            if axis == 1:
                F = qt.data.shape[-1]
                y2 = _hip_dequant_int8_channel(qt.data.view(-1, F), qt.scale,
                                               qt.original_dtype, axis=1)
                return y2.view(qt.data.shape)
            return _hip_dequant_int8_channel_nd(qt.data, qt.scale, qt.axis, qt.original_dtype)
        if qt.mode == "group":
            if qt.group_size is None:
                raise ValueError("INT8 group dequant needs qt.group_size")
            q = qt.data
            ax = qt.axis + q.dim() if qt.axis < 0 else qt.axis
            if not 0 <= ax < max(q.dim(), 1):
                raise IndexError(f"axis {qt.axis} out of range for a {q.dim()}-D tensor")
            F = q.shape[ax] if q.dim() else 1
            if F % qt.group_size != 0:
                raise ValueError(
                    f"group_size {qt.group_size} must evenly divide axis length {F}"
                )
            if q.dim() == 0 or ax == q.dim() - 1:
                y_grouped = _hip_dequant_int8_group(q.reshape(-1, qt.group_size), qt.scale,
                                                    qt.group_size, qt.original_dtype)
                return y_grouped.view(q.shape)
            # any other axis: strided groups, no movedim copies
            # (dequantizers.py:61-72 makes two full copies here)
            return _hip_dequant_int8_group_nd(q, qt.scale, ax, qt.group_size, qt.original_dtype)
        raise ValueError(f"Unsupported INT8 mode '{qt.mode}'")

    raise ValueError(f"No dequant kernel registered for dtype={qt.dtype}")
