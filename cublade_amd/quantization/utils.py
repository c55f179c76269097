"""Linear-layer replacement used by quantize_model (reference:
quantization/utils.py:8-68)."""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Type

import torch.nn as nn

__all__ = ["replace_linear_layers"]


def replace_linear_layers(
    module: nn.Module,
    target_class: Type[nn.Module],
    target_modules: Optional[List[str]] = None,
    exclude_modules: Optional[List[str]] = None,
    quant_kwargs: Optional[Dict[str, Any]] = None,
    _parent_name: str = "",
) -> None:
    """Recursively swap every nn.Linear under ``module`` for ``target_class``.

    A layer whose dotted name contains any ``exclude_modules`` substring is
    kept; when ``target_modules`` is given, only layers whose name contains
    one of its substrings are swapped. The new layer is built with the old
    layer's shape, bias presence and weight dtype, attached, then quantized
    from the old weight; the old bias parameter is carried over.
    """
    kwargs = quant_kwargs or {}
    excluded = exclude_modules or []
    for name, child in list(module.named_children()):
        dotted = f"{_parent_name}.{name}" if _parent_name else name
        if not isinstance(child, nn.Linear):
            replace_linear_layers(child, target_class, target_modules, exclude_modules,
                                  quant_kwargs, _parent_name=dotted)
            continue
        if any(e in dotted for e in excluded):
            continue
        if target_modules is not None and not any(t in dotted for t in target_modules):
            continue
        old_weight, old_bias = child.weight, child.bias
        layer = target_class(child.in_features, child.out_features, bias=old_bias is not None,
                             dtype=old_weight.dtype, **kwargs)
        setattr(module, name, layer)
        layer.quantize(old_weight)
        if old_bias is not None:
            layer.bias = old_bias
