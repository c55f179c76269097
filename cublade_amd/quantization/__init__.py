"""Public quantization API, same names as cublade.quantization
(reference: quantization/__init__.py:1-17)."""
from .utils import *  # noqa: F401,F403  (replace_linear_layers, as in the reference)
from .tensor import QuantizedTensor
from .dequantizers import dequantize_tensor
from .linear import cuBladeW8A16LinearLayer, cubladeW8A16LinearLayer
from .quantizers import quantize_tensor, quantize_model
from .outlier_utils import (detect_activation_outlier_columns, detect_outlier_columns,
                            separate_outliers, split_weights_by_outliers)

__all__ = [
    "quantize_model",
    "quantize_tensor",
    "dequantize_tensor",
    "QuantizedTensor",
    "cuBladeW8A16LinearLayer",
    "cubladeW8A16LinearLayer",
    "detect_outlier_columns",
    "detect_activation_outlier_columns",
    "separate_outliers",
    "split_weights_by_outliers",
]
