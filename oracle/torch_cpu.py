"""Per-tensor INT8 / FP8 quant and dequant as multi-threaded torch CPU ops
(TEST INFRASTRUCTURE ONLY: the CPU baseline of bench.py, which may import
it, as may tests/; nothing under cublade_amd/ does).

The same formulas as the C oracle (cbq_oracle.c), written with torch tensor
ops so that a whole config tensor runs on every host core:
  amax  = max |x| over the float32-widened input, NaN ignored
          (quantize_int8.cu:47-101, quantize_per_tensor_fp8.cu:38-86 fold with fmaxf)
  inv   = fp32(Q / max(amax, fp32(eps)))  (quantize_int8.cu:120-126; IEEE
          division, the reference FP8 module's intent, :99-102)
  INT8  q = clamp(round_half_even(fp32(x * inv)), -127, 127), NaN -> 0
          (int8_pack.cuh:51-56)
  FP8   q = e4m3fn(clamp(fp32(x * inv), -448, 448)), NaN kept
          (quantize_per_tensor_fp8.cu:117,129, __NV_SATFINITE)
  scale = fp32(1 / inv)
  dequant y = T(fp32(q) * scale)           (dequantize_int8.cu:29-64,
          dequantize_per_tensor_fp8.cu:23-66)
tests/test_oracle_golden.py pins these against the C oracle bit for bit.
"""
from __future__ import annotations

import torch

_QMAX = {torch.int8: 127.0, torch.float8_e4m3fn: 448.0}


def quant_tensor(x: torch.Tensor, dtype: torch.dtype, eps: float = 1e-12):
    """(codes, scale): codes like x in `dtype`, scale a 0-d float32."""
    f = x.float()
    a = f.abs()
    a = torch.where(torch.isnan(a), torch.zeros((), dtype=a.dtype), a)
    amax = a.amax() if a.numel() else torch.zeros(())
    qmax = torch.tensor(_QMAX[dtype], dtype=torch.float32)
    inv = qmax / torch.maximum(amax, torch.tensor(eps, dtype=torch.float32))
    v = f * inv
    if dtype == torch.int8:
        r = torch.round(v).clamp(-127.0, 127.0)
        q = torch.where(torch.isnan(r), torch.zeros((), dtype=r.dtype), r).to(torch.int8)
    else:
        q = v.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    scale = torch.tensor(1.0, dtype=torch.float32) / inv
    return q, scale


def dequant_tensor(q: torch.Tensor, scale: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    return (q.float() * scale).to(out_dtype)
