"""Thin wrappers over the HIP C ABI (libcublade_quant.so).

``bindings.hip`` takes the place of the reference's ``cublade.bindings.cuda``
quantization wrappers (same function names, signatures and defaults) and of
the ``cublade.bindings.triton.matmul`` call the W8A16 layer made.
"""
from . import hip

__all__ = ["hip"]
