"""W8A16 linear on the HIP C ABI: the one-launch replacement of the reference
forward chain (quantization/linear.py:94-135: int8 -> activation copy,
triton_matmul via bindings/triton/matmul.py:17-132, * scales, outlier
side-GEMM, + bias)."""
from __future__ import annotations

import torch

from ... import _abi


def w8a16_linear(
    x2d: torch.Tensor,
    int8_weights: torch.Tensor,
    scales: torch.Tensor,
    bias: torch.Tensor | None = None,
    outlier_cols: torch.Tensor | None = None,
    outlier_weights: torch.Tensor | None = None,
) -> torch.Tensor:
    """y = (x2d @ int8_weights.T) * scales + x2d[:, oc] @ outlier_weights.T + bias.

    Args:
        x2d: [M, K] contiguous CUDA (HIP) activations, fp16 / bf16 (MFMA path)
            or fp32 (general path).
        int8_weights: [N, K] int8, contiguous, on x2d's device. Outlier
            columns (if any) must hold 0.
        scales: [N] per-output-channel scales (converted to x2d's dtype, as
            the reference does with ``self.scales.to(dtype=x2d.dtype)``).
        bias: optional [N] (converted to x2d's dtype).
        outlier_cols: optional int64 [n_out] column indices into K.
        outlier_weights: [N, n_out] weights of those columns (converted to
            x2d's dtype).

    Returns:
        y: [M, N] in x2d's dtype, fp32 accumulation, one final rounding.
    """
    if not x2d.is_cuda:
        raise RuntimeError("w8a16_linear: x must be on CUDA")
    if x2d.dim() != 2:
        raise RuntimeError("w8a16_linear: x must be 2-D [M, K]")
    if x2d.dtype not in _abi.DTYPE_CODE:
        raise RuntimeError(f"w8a16_linear: unsupported activation dtype {x2d.dtype}")
    dev, dt = x2d.device, x2d.dtype
    x2d = x2d.contiguous()
    M, K = x2d.shape
    if int8_weights.dtype != torch.int8 or int8_weights.dim() != 2 or int8_weights.size(1) != K:
        raise RuntimeError(f"w8a16_linear: int8_weights must be int8 [N, {K}], got "
                           f"{tuple(int8_weights.shape)} {int8_weights.dtype}")
    N = int8_weights.size(0)
    wq = int8_weights.to(device=dev).contiguous()
    s = scales.to(device=dev, dtype=dt).contiguous()
    if s.numel() != N:
        raise RuntimeError(f"w8a16_linear: scales must have {N} elements")
    b = None
    if bias is not None:
        b = bias.to(device=dev, dtype=dt).contiguous()
        if b.numel() != N:
            raise RuntimeError(f"w8a16_linear: bias must have {N} elements")
    n_out = 0
    oc = wo = None
    if outlier_cols is not None and outlier_cols.numel() > 0:
        oc = outlier_cols.to(device=dev, dtype=torch.int64).contiguous()
        n_out = oc.numel()
        if outlier_weights is None:
            raise RuntimeError("w8a16_linear: outlier_cols given without outlier_weights")
        wo = outlier_weights.to(device=dev, dtype=dt).contiguous()
        if tuple(wo.shape) != (N, n_out):
            raise RuntimeError(f"w8a16_linear: outlier_weights must be [{N}, {n_out}]")
    y = torch.empty((M, N), dtype=dt, device=dev)
    if M == 0 or N == 0:
        return y
    L = _abi.lib()
    with _abi.on_device(dev):
        ws = _abi.workspace(dev, L.cbq_w8a16_ws_bytes(M, N, K, n_out, _abi.DTYPE_CODE[dt]))
        rc = L.cbq_w8a16_linear(_abi.ptr(x2d), _abi.DTYPE_CODE[dt], _abi.ptr(wq), _abi.ptr(s),
                                _abi.ptr(b), _abi.ptr(oc), n_out, _abi.ptr(wo), M, N, K,
                                _abi.ptr(ws), ws.numel(), _abi.ptr(y), _abi.stream_handle(dev))
    _abi.check(rc, "w8a16_linear")
    return y
