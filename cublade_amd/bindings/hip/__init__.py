"""HIP bindings of the quantization hot path (one module per reference module:
bindings/cuda/{quantize,dequantize}_{fp8,int8}.py), the W8A16 linear, and the
dense GEMM of bindings/cuda/wmma.py."""
from .quantize_fp8 import quantize_per_tensor_fp8
from .dequantize_fp8 import dequantize_per_tensor_fp8
from .quantize_int8 import (
    quantize_per_tensor_int8,
    quantize_per_channel_int8,
    quantize_per_group_int8,
)
from .dequantize_int8 import (
    dequantize_per_tensor_int8,
    dequantize_per_channel_int8,
    dequantize_per_group_int8,
)
from .w8a16 import w8a16_linear
from .wmma import wmma_gemm

__all__ = [
    "quantize_per_tensor_fp8",
    "dequantize_per_tensor_fp8",
    "quantize_per_tensor_int8",
    "quantize_per_channel_int8",
    "quantize_per_group_int8",
    "dequantize_per_tensor_int8",
    "dequantize_per_channel_int8",
    "dequantize_per_group_int8",
    "w8a16_linear",
    "wmma_gemm",
]
