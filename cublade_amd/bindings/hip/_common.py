"""Argument checks shared by the HIP binding wrappers.

They restate the reference's kernel-level TORCH_CHECKs (raised there as
RuntimeError) so that the bindings fail the same way:
``quantize_per_tensor_fp8.cu:164-167``, ``quantize_int8.cu:450-460``,
``dequantize_per_tensor_fp8.cu:88-97``, ``dequantize_int8.cu:191-202``.
"""
from __future__ import annotations

import torch

from ... import _abi


def check_cuda_contig(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on CUDA")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def check_float_input(x: torch.Tensor, allow_f32: bool) -> int:
    check_cuda_contig(x, "x")
    if x.dtype == torch.float16 or x.dtype == torch.bfloat16 or (allow_f32 and x.dtype == torch.float32):
        return _abi.DTYPE_CODE[x.dtype]
    if allow_f32:
        raise RuntimeError("x must be torch.float16, torch.bfloat16, or torch.float32")
    raise RuntimeError("x must be torch.float16 or torch.bfloat16")


def check_scale(scale: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    if not scale.is_cuda:
        raise RuntimeError("scale must be on CUDA")
    if scale.dtype != torch.float32:
        raise RuntimeError("scale must be torch.float32")
    if scale.device != q.device:
        raise RuntimeError("scale must be on the same device as q")
    return scale.contiguous()


def check_out_dtype(dtype: torch.dtype) -> int:
    if dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("out_dtype must be torch.float16 or torch.bfloat16")
    return _abi.DTYPE_CODE[dtype]
