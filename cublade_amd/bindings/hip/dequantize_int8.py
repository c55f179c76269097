"""Symmetric INT8 dequantization per tensor / channel / group (reference:
bindings/cuda/dequantize_int8.py:18-79, kernels/cuda/quantization/dequantize_int8.cu:210-273)."""
from __future__ import annotations

import torch

from ... import _abi
from ._common import check_cuda_contig, check_out_dtype, check_scale


def _check_q(q: torch.Tensor) -> None:
    check_cuda_contig(q, "q")
    if q.dtype != torch.int8:
        raise RuntimeError("q must be torch.int8")


def dequantize_per_tensor_int8(
    q: torch.Tensor,
    scale: torch.Tensor,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """y = (float(q) * scale).to(dtype), one fp32 scale for the tensor."""
    _check_q(q)
    scale = check_scale(scale, q)
    out = check_out_dtype(dtype)
    if scale.numel() != 1:
        raise RuntimeError("scale must be a scalar for per-tensor mode")
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    n = q.numel()
    if n == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q.device):
        rc = L.cbq_dequant_int8_tensor(_abi.ptr(q), _abi.ptr(scale), n, _abi.ptr(y), out,
                                       _abi.stream_handle(q.device))
    _abi.check(rc, "dequantize_per_tensor_int8")
    return y


def dequantize_per_channel_int8(
    q: torch.Tensor,
    scale: torch.Tensor,
    dtype: torch.dtype = torch.bfloat16,
    axis: int = 0,
) -> torch.Tensor:
    """Per-channel dequantization of q viewed as (C, F). axis=0: scale (C,)
    (reference); axis=1 (extension): scale (F,). F need not be a multiple of 8."""
    _check_q(q)
    scale = check_scale(scale, q)
    out = check_out_dtype(dtype)
    if q.dim() < 1:
        raise RuntimeError("q must have at least 1 dim")
    if axis not in (0, 1):
        raise RuntimeError(f"axis must be 0 or 1, got {axis}")
    C = q.size(0)
    F = q.numel() // C if C else 0
    if axis == 0 and scale.numel() != C:
        raise RuntimeError("scale must have C elements (size(0) of q)")
    if axis == 1 and scale.numel() != F:
        raise RuntimeError("scale must have F elements (numel(q) / size(0)) for axis 1")
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    if C == 0 or F == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q.device):
        rc = L.cbq_dequant_int8_channel(_abi.ptr(q), _abi.ptr(scale), C, F, axis, _abi.ptr(y),
                                        out, _abi.stream_handle(q.device))
    _abi.check(rc, "dequantize_per_channel_int8")
    return y


def dequantize_per_group_int8(
    q_grouped: torch.Tensor,
    scale: torch.Tensor,
    group_size: int,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Per-group dequantization of a (num_groups, group_size) int8 tensor with
    scale (num_groups,)."""
    _check_q(q_grouped)
    scale = check_scale(scale, q_grouped)
    out = check_out_dtype(dtype)
    if q_grouped.dim() != 2:
        raise RuntimeError("q_grouped must be 2D (num_groups, group_size)")
    if q_grouped.size(1) != group_size:
        raise RuntimeError("q_grouped.size(1) must equal group_size")
    if not (0 < group_size <= 4096):
        raise RuntimeError("group_size must be in (0, 4096]")
    G = q_grouped.size(0)
    if scale.numel() != G:
        raise RuntimeError("scale must have num_groups elements")
    y = torch.empty(q_grouped.shape, dtype=dtype, device=q_grouped.device)
    if G == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q_grouped.device):
        rc = L.cbq_dequant_int8_group(_abi.ptr(q_grouped), _abi.ptr(scale), G, int(group_size),
                                      _abi.ptr(y), out, _abi.stream_handle(q_grouped.device))
    _abi.check(rc, "dequantize_per_group_int8")
    return y


def dequantize_per_channel_int8_nd(
    q: torch.Tensor,
    scale: torch.Tensor,
    axis: int,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Per-channel dequantization along any axis (scale (q.size(axis),)),
    without copies; an extension of the reference's axis-0 mode."""
    from .quantize_int8 import _axis_view
    _check_q(q)
    scale = check_scale(scale, q)
    out = check_out_dtype(dtype)
    if q.dim() < 1:
        raise RuntimeError("q must have at least 1 dim")
    axis = axis + q.dim() if axis < 0 else axis
    if not 0 <= axis < q.dim():
        raise RuntimeError(f"axis {axis} out of range for a {q.dim()}-D tensor")
    outer, C, inner = _axis_view(q.shape, axis)
    if scale.numel() != C:
        raise RuntimeError(f"scale must have {C} elements (size({axis}) of q)")
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    if q.numel() == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q.device):
        rc = L.cbq_dequant_int8_channel_nd(_abi.ptr(q), _abi.ptr(scale), outer, C, inner,
                                           _abi.ptr(y), out, _abi.stream_handle(q.device))
    _abi.check(rc, "dequantize_per_channel_int8_nd")
    return y


def dequantize_per_group_int8_nd(
    q: torch.Tensor,
    scale: torch.Tensor,
    axis: int,
    group_size: int,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Per-group dequantization with groups along any axis (scales in the
    reference's movedim order), without the copies of dequantizers.py:58-72."""
    from .quantize_int8 import _axis_view
    _check_q(q)
    scale = check_scale(scale, q)
    out = check_out_dtype(dtype)
    axis = axis + q.dim() if axis < 0 else axis
    if not 0 <= axis < q.dim():
        raise RuntimeError(f"axis {axis} out of range for a {q.dim()}-D tensor")
    if not 0 < group_size <= 4096:
        raise RuntimeError(f"group_size must be in (0, 4096], got {group_size}")
    outer, Lq, inner = _axis_view(q.shape, axis)
    if Lq % group_size != 0:
        raise RuntimeError(f"group_size {group_size} must evenly divide axis length {Lq}")
    ng = outer * inner * (Lq // group_size)
    if scale.numel() != ng:
        raise RuntimeError(f"scale must have {ng} elements (one per group)")
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    if ng == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q.device):
        ws = _abi.workspace(q.device,
                            L.cbq_dequant_int8_group_nd_ws_bytes(outer, Lq, inner, group_size))
        rc = L.cbq_dequant_int8_group_nd(_abi.ptr(q), _abi.ptr(scale), outer, Lq, inner,
                                         group_size, _abi.ptr(ws), ws.numel(), _abi.ptr(y), out,
                                         _abi.stream_handle(q.device))
    _abi.check(rc, "dequantize_per_group_int8_nd")
    return y
