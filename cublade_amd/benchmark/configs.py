"""Seeded synthetic inputs of the BASELINE configurations (CPU-generated with
torch.Generator, then moved to the device by the caller).

C1  FP8 per tensor:   bf16 [4096, 4096] ~ N(0, 1), seed 0
C2  INT8 per tensor:  fp16 [8192, 8192] = 0.5 * Student-t(df=3), seed 1
C3  INT8 per channel: bf16 [28672, 8192] ~ N(0, 0.02), 8 columns x 20, seed 2
C4  INT8 per group:   bf16 [16384, 14336] ~ N(0, 1) * U[0.1, 10] per row, seed 3
C5  W8A16 linear:     fp16 x [M, 4096] ~ N(0, 1) with 6 feature columns at
                      sign * U(8, 20); W [11008, 4096] ~ N(0, 0.02), seed 4
"""
from __future__ import annotations

import torch


def c1_fp8_tensor() -> torch.Tensor:
    g = torch.Generator().manual_seed(0)
    return torch.randn(4096, 4096, generator=g).bfloat16()


def c2_int8_tensor() -> torch.Tensor:
    g = torch.Generator().manual_seed(1)
    shape = (8192, 8192)
    z = torch.randn(*shape, generator=g)
    c = [torch.randn(*shape, generator=g) for _ in range(3)]
    t = z / torch.sqrt((c[0] ** 2 + c[1] ** 2 + c[2] ** 2) / 3)
    x = (0.5 * t).half()
    assert torch.isfinite(x).all()
    return x


def c3_int8_channel() -> torch.Tensor:
    g = torch.Generator().manual_seed(2)
    w = 0.02 * torch.randn(28672, 8192, generator=g)
    cols = torch.randperm(8192, generator=g)[:8]
    w[:, cols] *= 20
    return w.bfloat16()


def c4_int8_group() -> torch.Tensor:
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16384, 14336, generator=g)
    x *= 0.1 + 9.9 * torch.rand(16384, 1, generator=g)
    return x.bfloat16()


def c5_w8a16(M: int):
    """Returns (x fp16 [M, 4096], W fp16 [11008, 4096])."""
    g = torch.Generator().manual_seed(4)
    K, N = 4096, 11008
    x = torch.randn(M, K, generator=g)
    oc = torch.sort(torch.randperm(K, generator=g)[:6]).values
    mag = 8.0 + 12.0 * torch.rand(M, 6, generator=g)
    x[:, oc] = torch.sign(torch.randn(M, 6, generator=g)) * mag
    w = 0.02 * torch.randn(N, K, generator=g)
    return x.half(), w.half()
