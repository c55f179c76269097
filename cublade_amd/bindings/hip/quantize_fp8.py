"""Per-tensor FP8 E4M3 quantization (reference: bindings/cuda/quantize_fp8.py:15-34,
kernels/cuda/quantization/quantize_per_tensor_fp8.cu:162-182)."""
from __future__ import annotations

import torch

from ... import _abi
from ._common import check_exchange, check_float_input


def quantize_per_tensor_fp8(
    x: torch.Tensor,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor symmetric FP8 (E4M3) quantization.

    Math (bit-exact to the reference kernels):
        amax  = max(|x|)                      (NaN inputs ignored)
        inv   = fp32(448 / max(amax, eps))
        q     = e4m3fn(x * inv), round to nearest even, saturated to +-448
        scale = fp32(1 / inv)                 (~= amax / 448)

    Args:
        x: torch.float16 or torch.bfloat16 contiguous CUDA (HIP) tensor.
        eps: floor on amax.

    Returns:
        (q, scale): q is float8_e4m3fn shaped like x; scale is a 0-d float32
        tensor on x's device (0 for an empty x).
    """
    code = check_float_input(x, allow_f32=False)
    dev = x.device
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=dev)
    n = x.numel()
    if n == 0:
        return q, torch.zeros((), dtype=torch.float32, device=dev)
    scale = torch.empty((), dtype=torch.float32, device=dev)
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_quant_tensor_ws_bytes())
        rc = L.cbq_quant_fp8_tensor(_abi.ptr(x), code, n, float(eps), _abi.ptr(ws), ws.numel(),
                                    _abi.ptr(q), _abi.ptr(scale), _abi.stream_handle(dev))
    _abi.check(rc, "quantize_per_tensor_fp8")
    check_exchange(dev, "quantize_per_tensor_fp8")
    return q, scale
