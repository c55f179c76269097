"""Argument checks shared by the HIP binding wrappers.

They restate the reference's kernel-level TORCH_CHECKs (raised there as
RuntimeError) so that the bindings fail the same way:
``quantize_per_tensor_fp8.cu:164-167``, ``quantize_int8.cu:450-460``,
``dequantize_per_tensor_fp8.cu:88-97``, ``dequantize_int8.cu:191-202``.
"""
from __future__ import annotations

import os

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


def check_exchange(dev: torch.device, what: str) -> None:
    """With CUBLADE_CHECK_EXCHANGE=1 in the environment: synchronise after a
    per-tensor quant and raise RuntimeError if its workgroups' exchange timed
    out (the status word of the stream's workspace; cleared before raising).
    Off by default, so that calls stay asynchronous; a timed-out call's scale
    is NaN whenever a code is not exact, and later calls are exact either way."""
    if os.environ.get("CUBLADE_CHECK_EXCHANGE", "") in ("", "0"):
        return
    if _abi.tensor_quant_status(dev):
        _abi.clear_tensor_quant_status(dev)
        raise RuntimeError(
            f"{what}: the workgroups of the one-launch per-tensor quant gave up waiting for "
            f"each other (exchange timed out; other work kept part of the grid off the GPU): "
            f"the result is not valid, repeat the call")
