"""cublade_amd - MI355X-native (gfx950) quantization hot path of cuBlade.

Drop-in for ``cublade.quantization``: quantize_tensor, dequantize_tensor,
QuantizedTensor, quantize_model, cuBladeW8A16LinearLayer and the outlier
utilities, backed by hand-written HIP kernels behind a C ABI
(include/cublade_quant.h, libcublade_quant.so).

Import-time warm-up as in the reference (cublade/__init__.py:9-32): skipped
with CUBLADE_SKIP_WARMUP=1 (or CUBLADE_POST_INSTALL_ACTIVE=1).
"""
import os as _os

from . import bindings
from .quantization import *  # noqa: F401,F403
from .quantization import __all__ as _quant_all

__all__ = ["bindings", *_quant_all]


def _maybe_compile() -> None:
    if _os.environ.get("CUBLADE_SKIP_WARMUP") == "1":
        return
    if _os.environ.get("CUBLADE_POST_INSTALL_ACTIVE") == "1":
        return
    try:
        from cublade_amd._post_install import main
        main()
    except Exception as e:  # the warm-up never blocks the import
        import sys as _sys
        print(f"[cublade] warm-up skipped: {e}", file=_sys.stderr)


_maybe_compile()
