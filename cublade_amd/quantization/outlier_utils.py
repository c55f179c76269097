"""LLM.int8-style outlier column utilities (reference:
quantization/outlier_utils.py:12-101). A column (input feature) of a
[out_features, in_features] weight is an outlier when any of its entries
exceeds the threshold in magnitude (strict >).

detect_activation_outlier_columns is an addition for the layer's opt-in
activation mode: LLM.int8's own criterion, applied to a batch of inputs,
where a feature is an outlier when any activation in it exceeds the
threshold."""
from __future__ import annotations

from typing import List, Tuple

import torch


def detect_outlier_columns(weight: torch.Tensor, threshold: float = 6.0) -> List[int]:
    """Indices (ascending) of the columns whose max |w| is > threshold."""
    col_peak = weight.abs().amax(dim=0)
    return torch.nonzero(col_peak > threshold).flatten().tolist()


def detect_activation_outlier_columns(x: torch.Tensor, threshold: float = 6.0) -> List[int]:
    """Indices (ascending) of the input features (last dimension of x) whose
    max |x| over every other dimension is > threshold (NaN never counts)."""
    peak = x.detach().reshape(-1, x.shape[-1]).abs().amax(dim=0)
    return torch.nonzero(peak > threshold).flatten().tolist()


def split_weights_by_outliers(
    weight: torch.Tensor, outlier_cols: List[int]
) -> Tuple[torch.Tensor, torch.Tensor, List[int], List[int]]:
    """Return (weight[:, normal], weight[:, outlier_cols], normal, outlier_cols)
    where normal lists the remaining columns in ascending order."""
    outliers = set(outlier_cols)
    normal_cols = [c for c in range(weight.shape[1]) if c not in outliers]
    return weight[:, normal_cols], weight[:, outlier_cols], normal_cols, outlier_cols


def separate_outliers(
    weight: torch.Tensor, threshold: float = 6.0
) -> Tuple[torch.Tensor, torch.Tensor, List[int], List[int]]:
    """detect_outlier_columns followed by split_weights_by_outliers."""
    return split_weights_by_outliers(weight, detect_outlier_columns(weight, threshold))
