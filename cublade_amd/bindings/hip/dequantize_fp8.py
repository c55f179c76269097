"""Per-tensor FP8 E4M3 dequantization (reference: bindings/cuda/dequantize_fp8.py:15-35,
kernels/cuda/quantization/dequantize_per_tensor_fp8.cu:84-109)."""
from __future__ import annotations

import torch

from ... import _abi
from ._common import check_cuda_contig, check_out_dtype, check_scale


def dequantize_per_tensor_fp8(
    q: torch.Tensor,
    scale: torch.Tensor,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Per-tensor FP8 (E4M3) dequantization: y = (float(q) * scale).to(dtype),
    rounded to nearest even.

    Args:
        q: torch.float8_e4m3fn contiguous CUDA (HIP) tensor.
        scale: 0-d or 1-element torch.float32 tensor on q's device.
        dtype: torch.float16 or torch.bfloat16 (default torch.bfloat16).
    """
    check_cuda_contig(q, "q")
    if q.dtype != torch.float8_e4m3fn:
        raise RuntimeError("q must be torch.float8_e4m3fn")
    scale = check_scale(scale, q)
    if scale.numel() != 1:
        raise RuntimeError("scale must be a 0-d or 1-element tensor")
    out = check_out_dtype(dtype)
    y = torch.empty(q.shape, dtype=dtype, device=q.device)
    n = q.numel()
    if n == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(q.device):
        rc = L.cbq_dequant_fp8_tensor(_abi.ptr(q), _abi.ptr(scale), n, _abi.ptr(y), out,
                                      _abi.stream_handle(q.device))
    _abi.check(rc, "dequantize_per_tensor_fp8")
    return y
