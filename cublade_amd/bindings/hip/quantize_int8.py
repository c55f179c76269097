"""Symmetric INT8 quantization per tensor / channel / group (reference:
bindings/cuda/quantize_int8.py:18-87, kernels/cuda/quantization/quantize_int8.cu:470-536)."""
from __future__ import annotations

import torch

from ... import _abi
from ._common import check_exchange, check_float_input


def quantize_per_tensor_int8(
    x: torch.Tensor,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor symmetric INT8 quantization.

    Math (bit-exact to the reference kernels):
        inv   = fp32(127 / max(amax, eps))
        q     = clamp(round_half_even(x * inv), -127, 127)
        scale = fp32(1 / inv)

    Args:
        x: contiguous CUDA (HIP) tensor, dtype fp16 / bf16 / fp32.

    Returns:
        (q, scale): int8 shaped like x, 0-d float32 scale (0 for an empty x).
    """
    code = check_float_input(x, allow_f32=True)
    dev = x.device
    q = torch.empty(x.shape, dtype=torch.int8, device=dev)
    n = x.numel()
    if n == 0:
        return q, torch.zeros((), dtype=torch.float32, device=dev)
    scale = torch.empty((), dtype=torch.float32, device=dev)
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_quant_tensor_ws_bytes())
        rc = L.cbq_quant_int8_tensor(_abi.ptr(x), code, n, float(eps), _abi.ptr(ws), ws.numel(),
                                     _abi.ptr(q), _abi.ptr(scale), _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_tensor_int8")
    check_exchange(dev, "quantize_per_tensor_int8")
    return q, scale


def quantize_per_channel_int8(
    x: torch.Tensor,
    eps: float = 1e-12,
    axis: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel symmetric INT8 quantization of x viewed as (C, F),
    C = x.size(0), F = numel / C.

    axis=0 (the reference's only mode): one scale per row, shape (C,).
    axis=1 (extension): one scale per column of that view, shape (F,); the
    same math with the maximum taken over rows.

    Unlike the reference (quantize_int8.cu:496-498), F need not be a multiple
    of 16 / element_size.
    """
    code = check_float_input(x, allow_f32=True)
    if x.dim() < 1:
        raise RuntimeError("x must have at least 1 dim for per-channel quant")
    if axis not in (0, 1):
        raise RuntimeError(f"axis must be 0 or 1, got {axis}")
    dev = x.device
    C = x.size(0)
    F = x.numel() // C if C else 0
    q = torch.empty(x.shape, dtype=torch.int8, device=dev)
    nscale = C if axis == 0 else F
    if C == 0 or F == 0:
        return q, torch.zeros((nscale,), dtype=torch.float32, device=dev)
    scale = torch.empty((nscale,), dtype=torch.float32, device=dev)
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_quant_int8_channel_ws_bytes(C, F, axis))
        rc = L.cbq_quant_int8_channel(_abi.ptr(x), code, C, F, axis, float(eps), _abi.ptr(ws),
                                      ws.numel(), _abi.ptr(q), _abi.ptr(scale),
                                      _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_channel_int8")
    return q, scale


def quantize_per_group_int8(
    x_grouped: torch.Tensor,
    group_size: int,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-group symmetric INT8 quantization of a (num_groups, group_size)
    contiguous tensor, 0 < group_size <= 4096. Returns (q int8 of the same
    shape, scale float32 (num_groups,))."""
    code = check_float_input(x_grouped, allow_f32=True)
    if x_grouped.dim() != 2:
        raise RuntimeError("x_grouped must be 2D (num_groups, group_size)")
    if x_grouped.size(1) != group_size:
        raise RuntimeError("x_grouped.size(1) must equal group_size")
    if not (0 < group_size <= 4096):
        raise RuntimeError("group_size must be in (0, 4096]")
    dev = x_grouped.device
    G = x_grouped.size(0)
    q = torch.empty(x_grouped.shape, dtype=torch.int8, device=dev)
    if G == 0:
        return q, torch.zeros((0,), dtype=torch.float32, device=dev)
    scale = torch.empty((G,), dtype=torch.float32, device=dev)
    L = _abi.lib()
    with _abi.on_device(dev):
        rc = L.cbq_quant_int8_group(_abi.ptr(x_grouped), code, G, int(group_size), float(eps),
                                    _abi.ptr(q), _abi.ptr(scale), _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_group_int8")
    return q, scale


def _axis_view(shape, axis: int) -> tuple[int, int, int]:
    """(outer, length, inner) of an N-D shape around `axis`."""
    outer = 1
    for d in shape[:axis]:
        outer *= int(d)
    inner = 1
    for d in shape[axis + 1:]:
        inner *= int(d)
    return outer, int(shape[axis]), inner


def quantize_per_channel_int8_nd(
    x: torch.Tensor,
    axis: int,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel symmetric INT8 quantization along any axis of a contiguous
    N-D tensor, without transposing copies: one scale per position of
    `axis`, the maximum taken over all other dims. Returns (q int8 of x's
    shape, scale float32 (x.size(axis),)). An extension of the reference,
    whose channel mode is axis 0 only (quantizers.py:116-121)."""
    code = check_float_input(x, allow_f32=True)
    if x.dim() < 1:
        raise RuntimeError("x must have at least 1 dim for per-channel quant")
    axis = axis + x.dim() if axis < 0 else axis
    if not 0 <= axis < x.dim():
        raise RuntimeError(f"axis {axis} out of range for a {x.dim()}-D tensor")
    dev = x.device
    outer, C, inner = _axis_view(x.shape, axis)
    q = torch.empty(x.shape, dtype=torch.int8, device=dev)
    if x.numel() == 0:
        return q, torch.zeros((C,), dtype=torch.float32, device=dev)
    scale = torch.empty((C,), dtype=torch.float32, device=dev)
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_quant_int8_channel_nd_ws_bytes(outer, C, inner))
        rc = L.cbq_quant_int8_channel_nd(_abi.ptr(x), code, outer, C, inner, float(eps),
                                         _abi.ptr(ws), ws.numel(), _abi.ptr(q), _abi.ptr(scale),
                                         _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_channel_int8_nd")
    return q, scale


def quantize_per_group_int8_nd(
    x: torch.Tensor,
    axis: int,
    group_size: int,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-group symmetric INT8 quantization with groups of `group_size`
    consecutive positions along any axis of a contiguous N-D tensor, without
    the reference's movedim / contiguous copies (quantizers.py:122-132).
    Returns (q int8 of x's shape, scale float32 (num_groups,)) with the
    scales in the reference's order (groups of x.movedim(axis, -1))."""
    code = check_float_input(x, allow_f32=True)
    axis = axis + x.dim() if axis < 0 else axis
    if not 0 <= axis < x.dim():
        raise RuntimeError(f"axis {axis} out of range for a {x.dim()}-D tensor")
    if not 0 < group_size <= 4096:
        raise RuntimeError(f"group_size must be in (0, 4096], got {group_size}")
    dev = x.device
    outer, Lx, inner = _axis_view(x.shape, axis)
    if Lx % group_size != 0:
        raise RuntimeError(f"group_size {group_size} must evenly divide axis length {Lx}")
    q = torch.empty(x.shape, dtype=torch.int8, device=dev)
    ng = outer * inner * (Lx // group_size)
    scale = torch.empty((ng,), dtype=torch.float32, device=dev)
    if ng == 0:
        return q, scale
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_quant_int8_group_nd_ws_bytes(outer, Lx, inner, group_size))
        rc = L.cbq_quant_int8_group_nd(_abi.ptr(x), code, outer, Lx, inner, group_size,
                                       float(eps), _abi.ptr(ws), ws.numel(), _abi.ptr(q),
                                       _abi.ptr(scale), _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_group_int8_nd")
    return q, scale
