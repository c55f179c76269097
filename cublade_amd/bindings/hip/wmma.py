"""Dense GEMM on the MI355X matrix cores, bound like the reference's
cublade.bindings.cuda.wmma (bindings/cuda/wmma.py:15-43, kernel and host
checks kernels/cuda/wmma.cu:29-261): same function name, arguments,
precision table and error messages."""
from __future__ import annotations

import torch

from ... import _abi

# input dtype -> (default accumulator, accepted accumulators); wmma.cu:201-258.
_ACC = {
    torch.float16: (torch.float32, (torch.float32, torch.float16)),
    torch.bfloat16: (torch.float32, (torch.float32,)),
    torch.int8: (torch.int32, (torch.int32,)),
    torch.uint8: (torch.int32, (torch.int32,)),
}
_ACC_ERR = {
    torch.float16: "float16 inputs support float32 or float16 accumulator",
    torch.bfloat16: "bfloat16 inputs only support float32 accumulator",
    torch.int8: "int8 inputs only support int32 accumulator",
    torch.uint8: "uint8 inputs only support int32 accumulator",
}


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _operand_b(B: torch.Tensor):
    """(tensor, layout): a contiguous [K, N] B is read as stored; the
    transposed view of a contiguous [N, K] tensor (B = W.t()) is read in
    place as B^T; any other layout is made contiguous first."""
    if B.is_contiguous():
        return B, _abi.MM_B_KN
    if B.t().is_contiguous():
        return B, _abi.MM_B_NK
    return B.contiguous(), _abi.MM_B_KN


def mm(A: torch.Tensor, B: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """C = A @ B on the MFMA kernels for any M, N, K that are multiples of 16.

    A: [M, K]; B: [K, N] (contiguous, or the transposed view of a contiguous
    [N, K] weight, which is not copied). int8 / uint8 -> int32 (exact modulo
    2^32), fp16 -> fp32 or fp16, bf16 -> fp32 (fp32 accumulation, one
    rounding). Raises RuntimeError on invalid arguments.
    """
    if A.dtype not in _ACC:
        raise RuntimeError("Unsupported dtype. Expected: float16, bfloat16, int8, or uint8")
    default, accepted = _ACC[A.dtype]
    out = default if out_dtype is None else out_dtype
    if out not in accepted:
        raise RuntimeError(_ACC_ERR[A.dtype])
    M, K = A.shape
    N = B.shape[1]
    A = A if A.is_contiguous() else A.contiguous()
    Bt, layout = _operand_b(B)
    if not _aligned16(A):
        A = A.clone()
    if not _aligned16(Bt):
        Bt = Bt.clone() if layout == _abi.MM_B_KN else Bt.t().clone().t()
    C = torch.empty((M, N), dtype=out, device=A.device)
    if M == 0 or N == 0:
        return C
    L = _abi.lib()
    code = _abi.MM_DTYPE_CODE[A.dtype]
    with _abi.on_device(A.device):
        ws = _abi.workspace(A.device, L.cbq_mm_ws_bytes(M, N, K, code, layout))
        _abi.check(L.cbq_mm(_abi.ptr(A), _abi.ptr(Bt), code, layout, M, N, K, _abi.ptr(C),
                            _abi.MM_DTYPE_CODE[out], _abi.ptr(ws), ws.numel(),
                            _abi.stream_handle(A.device)), "wmma_gemm")
    return C


def wmma_gemm(
    A: torch.Tensor,
    B: torch.Tensor,
    acc_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Multi-precision GEMM C = A @ B (the reference's WMMA 16x16x16 GEMM,
    here on 32 x 32 MFMA tiles).

    Supported precision combinations:
        | Input dtype | Accumulator dtype |
        |-------------|-------------------|
        | float16     | float32 (default) |
        | float16     | float16           |
        | bfloat16    | float32           |
        | int8        | int32             |
        | uint8       | int32             |

    Args:
        A: Input matrix (M x K)
        B: Input matrix (K x N), must match A's dtype
        acc_dtype: Optional accumulator dtype. If None, uses default for input type.

    Returns:
        C: Output matrix (M x N) with accumulator dtype. Integer results are
        exact modulo 2^32; float16 accumulators are fp32 sums rounded once.

    Note:
        Dimensions M, N, K must be multiples of 16 (the reference's WMMA tile
        constraint, kept for drop-in behaviour).
    """
    if not (A.is_cuda and B.is_cuda):
        raise RuntimeError("Inputs must be CUDA tensors")
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("Inputs must be 2D matrices")
    if A.size(1) != B.size(0):
        raise RuntimeError("Matrix dimensions incompatible for GEMM")
    if A.dtype != B.dtype:
        raise RuntimeError("A and B must have the same dtype")
    M, K = A.shape
    N = B.shape[1]
    if M % 16 or N % 16 or K % 16:
        raise RuntimeError("Dimensions must be multiples of 16 for WMMA")
    return mm(A, B, acc_dtype)
