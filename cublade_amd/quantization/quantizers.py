"""quantize_tensor / quantize_model (reference: quantization/quantizers.py:22-224).

Same signatures, registry, defaults and exception types as the reference.
Backed by the HIP C ABI through ``cublade_amd.bindings.hip``. Two extensions:
``mode="channel"`` accepts any ``ch_axis`` (one scale per position of that
axis; the reference raises NotImplementedError for every ch_axis != 0), and
``mode="group"`` along a non-last axis runs in place (the reference moves
the axis last with two full copies; codes and scale order are the same).
An out-of-range ``ch_axis`` raises IndexError, as torch's movedim does in the
reference's group path.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn as nn

from .tensor import QuantizedTensor
from .utils import replace_linear_layers
from cublade_amd.bindings.hip.quantize_fp8 import (
    quantize_per_tensor_fp8 as _hip_quant_fp8_tensor,
)
from cublade_amd.bindings.hip.quantize_int8 import (
    quantize_per_tensor_int8 as _hip_quant_int8_tensor,
    quantize_per_channel_int8 as _hip_quant_int8_channel,
    quantize_per_group_int8 as _hip_quant_int8_group,
    quantize_per_channel_int8_nd as _hip_quant_int8_channel_nd,
    quantize_per_group_int8_nd as _hip_quant_int8_group_nd,
)

# (mode, storage dtype) -> kernel wrapper (quantizers.py:22-27).
_HIP_QUANT_KERNELS = {
    ("tensor", torch.float8_e4m3fn): _hip_quant_fp8_tensor,
    ("tensor", torch.int8): _hip_quant_int8_tensor,
    ("channel", torch.int8): _hip_quant_int8_channel,
    ("group", torch.int8): _hip_quant_int8_group,
}
# Reference name of the same table.
_CUDA_QUANT_KERNELS = _HIP_QUANT_KERNELS

# Accepted input dtypes per (mode, dtype) (quantizers.py:32-37): FP8 takes
# fp16/bf16; INT8 also takes fp32 (nn.Linear weights default to fp32).
_ALLOWED_INPUT_DTYPES = {
    ("tensor", torch.float8_e4m3fn): {torch.float16, torch.bfloat16},
    ("tensor", torch.int8): {torch.float16, torch.bfloat16, torch.float32},
    ("channel", torch.int8): {torch.float16, torch.bfloat16, torch.float32},
    ("group", torch.int8): {torch.float16, torch.bfloat16, torch.float32},
}


def _require_cuda_input(x: torch.Tensor, key, *, what: str) -> None:
    """Device / layout / dtype checks (quantizers.py:40-50). On ROCm a HIP
    tensor reports ``is_cuda``."""
    if not x.is_cuda:
        raise ValueError(f"{what}: tensor must be on CUDA, got device={x.device}")
    if not x.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    allowed = _ALLOWED_INPUT_DTYPES[key]
    if x.dtype not in allowed:
        names = sorted(str(d) for d in allowed)
        raise ValueError(f"{what}: tensor dtype must be one of {names}, got {x.dtype}")


_ZERO_POINTS: dict = {}


def _zero_scalar(device: torch.device) -> torch.Tensor:
    """The 0-d fp32 zero point of the symmetric scheme. One tensor per device
    is shared by QuantizedTensors (do not modify it in place), so a quantize
    call launches no fill kernel for it (the reference allocates a fresh
    torch.zeros(()) per call, quantizers.py:53-54). It is created and cached
    only outside graph capture (a fill recorded in a capture runs at replay
    time), and replaced by a fresh zero if it was modified in place (its
    version counter moved)."""
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
    entry = _ZERO_POINTS.get(key)
    if entry is not None and entry[0]._version == entry[1]:
        return entry[0]
    z = torch.zeros((), dtype=torch.float32, device=device)
    if not torch.cuda.is_current_stream_capturing():
        _ZERO_POINTS[key] = (z, z._version)
    return z


def channel_kernel_axis(ndim: int, ch_axis: int) -> int:
    """Map a user ``ch_axis`` to the channel kernel path: 0 -> one scale per
    row of the (size(0), numel/size(0)) view; 1 -> the last axis of an N-D
    tensor (N >= 2), one scale per column of the (numel/F, F) view; 2 -> any
    other axis, the N-D kernel on the (outer, C, inner) view. The reference
    supports axis 0 only (quantizers.py:116-121); the others are extensions
    without transposing copies."""
    ax = ch_axis + ndim if ch_axis < 0 else ch_axis
    if not 0 <= ax < max(ndim, 1):
        raise IndexError(f"ch_axis {ch_axis} out of range for a {ndim}-D tensor")
    if ax == 0:
        return 0
    if ax == ndim - 1:
        return 1
    return 2


def quantize_tensor(
    x: torch.Tensor,
    scheme: str = "symmetric",
    dtype: torch.dtype = torch.int8,
    mode: str = "tensor",
    group_size: int = 32,
    ch_axis: int = 0,
    eps: float = 1e-12,
) -> QuantizedTensor:
    """Quantize ``x`` per tensor, channel or group (symmetric only).

    x must be a contiguous CUDA (HIP) tensor: fp16 / bf16 for FP8, fp16 /
    bf16 / fp32 for INT8. FP8 supports mode "tensor" only. Returns a
    QuantizedTensor with a 0-d fp32 zero point.
    """
    if scheme != "symmetric":
        raise NotImplementedError(
            f"quantize_tensor: only scheme='symmetric' is supported, got '{scheme}'"
        )
    key = (mode, dtype)
    kernel = _HIP_QUANT_KERNELS.get(key)
    if kernel is None:
        raise ValueError(f"No quant kernel registered for mode='{mode}', dtype={dtype}")
    _require_cuda_input(x, key, what="quantize_tensor")

    if mode == "tensor":
        q, scale = kernel(x, eps)
    elif mode == "channel":
        axis = channel_kernel_axis(x.dim(), ch_axis)
        if axis == 0:
            q, scale = kernel(x, eps)
        elif axis == 1:
            F = x.shape[-1]
            q2, scale = kernel(x.view(-1, F), eps, axis=1)
            q = q2.view(x.shape)
        else:
            q, scale = _hip_quant_int8_channel_nd(x, ch_axis, eps)
    elif mode == "group":
        ax = ch_axis + x.dim() if ch_axis < 0 else ch_axis
        if not 0 <= ax < max(x.dim(), 1):
            raise IndexError(f"ch_axis {ch_axis} out of range for a {x.dim()}-D tensor")
        F = x.shape[ax] if x.dim() else 1
        if F % group_size != 0:
            raise ValueError(f"group_size {group_size} must evenly divide axis length {F}")
        if x.dim() == 0 or ax == x.dim() - 1:
            # groups along the last axis are contiguous rows
            q_grouped, scale = kernel(x.reshape(-1, group_size), group_size, eps)
            q = q_grouped.view(x.shape)
        else:
            # any other axis: strided groups, no movedim copies
            # (quantizers.py:123-132 makes two full copies here)
            q, scale = _hip_quant_int8_group_nd(x, ax, group_size, eps)
    else:
        raise ValueError(f"Unsupported mode '{mode}'; expected tensor / channel / group")

    return QuantizedTensor(q, scale, _zero_scalar(x.device), mode, ch_axis, group_size, dtype,
                           x.dtype)


QUANT_LAYER_REGISTRY = {}


def _init_registry():
    """Filled lazily (the layer module imports this one)."""
    if not QUANT_LAYER_REGISTRY:
        from .linear import cuBladeW8A16LinearLayer
        QUANT_LAYER_REGISTRY["w8a16"] = cuBladeW8A16LinearLayer


def quantize_model(
    model: nn.Module,
    quant_type: str = "w8a16",
    target_modules: Optional[List[str]] = None,
    exclude_modules: Optional[List[str]] = None,
    inplace: bool = True,
    **quant_kwargs,
):
    """Replace the model's nn.Linear layers with quantized layers
    (reference: quantizers.py:152-224).

    quant_type: "w8a16" (INT8 per-output-channel weights, 16-bit activations).
    target_modules / exclude_modules: substring filters on dotted names.
    inplace=False quantizes a deep copy. quant_kwargs go to the layer
    (handle_outliers, outlier_threshold). Returns the (possibly copied) model.
    """
    _init_registry()
    if quant_type not in QUANT_LAYER_REGISTRY:
        available = ", ".join(QUANT_LAYER_REGISTRY.keys())
        raise ValueError(f"Unknown quant_type '{quant_type}'. Available: {available}")
    if not inplace:
        from copy import deepcopy
        model = deepcopy(model)
    replace_linear_layers(
        model,
        target_class=QUANT_LAYER_REGISTRY[quant_type],
        target_modules=target_modules,
        exclude_modules=exclude_modules,
        quant_kwargs=quant_kwargs,
    )
    return model
