"""QuantizedTensor record (reference: quantization/tensor.py:5-14)."""
from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class QuantizedTensor:
    """Quantized data plus the metadata needed to dequantize it.

    data: int8 or float8_e4m3fn codes; scale: fp32 (0-d for mode "tensor",
    one per channel / group otherwise); zero_point: 0-d fp32 zero (symmetric
    only); mode: "tensor" | "channel" | "group"; axis: the ch_axis given at
    quantization; group_size: as given; dtype: storage dtype;
    original_dtype: dtype of the quantized input (dequant output dtype).
    """
    data: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor
    mode: str
    axis: int
    group_size: Optional[int]
    dtype: torch.dtype
    original_dtype: torch.dtype
