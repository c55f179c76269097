"""Generate the committed golden vectors in tests/golden/golden.npz.

The expected outputs here are computed with torch CPU tensor ops (fp32
division, ``torch.round`` half-to-even, ``Tensor.to(torch.float8_e4m3fn)``,
``Tensor.to(torch.bfloat16/float16)``) and float64 matmuls: an implementation
written independently of ``oracle/cbq_oracle.c``, so that comparing the two
pins the oracle. The formulas restate the reference kernels:

* per-tensor FP8: ``quantize_per_tensor_fp8.cu:88-132`` (inv = 448/max(amax,
  eps), q = satfinite_e4m3(x*inv), scale = 1/inv) and
  ``dequantize_per_tensor_fp8.cu:23-66``;
* INT8 tensor/channel/group: ``quantize_int8.cu:103-166, 232-297, 345-371``
  (inv = 127/max(amax, eps), q = clamp(rne(x*inv), +-127), scale = 1/inv) and
  ``dequantize_int8.cu:29-134``;
* W8A16: ``linear.py:97-135`` in exact (float64) accumulation.

Inputs follow the case lists of the reference demos
(``examples/quantization/quant_dequant_fp8.py:48-58``,
``examples/quantization/quant_dequant_int8.py:134-173``) at reduced sizes so
the fixture stays small.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "golden.npz"
EPS = torch.tensor(1e-12, dtype=torch.float32)
CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float8_e4m3fn:
        return t.contiguous().view(torch.uint8).numpy().copy()
    return t.contiguous().numpy().copy()


def inv_and_scale(amax: torch.Tensor, qmax: float):
    inv = torch.tensor(qmax, dtype=torch.float32) / torch.maximum(amax, EPS)
    scale = torch.tensor(1.0, dtype=torch.float32) / inv
    return inv, scale


def t_quant_fp8(x):
    xf = x.float()
    if xf.numel() == 0:
        return xf.to(torch.float8_e4m3fn), torch.tensor(0.0)
    inv, scale = inv_and_scale(xf.abs().max(), 448.0)
    q = (xf * inv).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale


def t_round_int8(v):
    return torch.round(v).clamp(-127, 127).to(torch.int8)


def t_quant_int8_tensor(x):
    xf = x.float()
    if xf.numel() == 0:
        return xf.to(torch.int8), torch.tensor(0.0)
    inv, scale = inv_and_scale(xf.abs().max(), 127.0)
    return t_round_int8(xf * inv), scale


def t_quant_int8_channel(x, axis):
    rows = x.shape[0]
    xf = x.float().reshape(rows, -1)
    if axis == 1:
        xf = xf.t()
    amax = xf.abs().amax(dim=1) if xf.shape[1] else torch.zeros(xf.shape[0])
    inv, scale = inv_and_scale(amax, 127.0)
    if xf.shape[1] == 0:
        scale = torch.zeros_like(scale)
    q = t_round_int8(xf * inv[:, None])
    if axis == 1:
        q = q.t()
    return q.contiguous().reshape(x.shape), scale


def t_quant_int8_group(x, g):
    xf = x.float().reshape(-1, g)
    inv, scale = inv_and_scale(xf.abs().amax(dim=1), 127.0)
    return t_round_int8(xf * inv[:, None]).reshape(x.shape), scale


def t_dequant(qf: torch.Tensor, scale_b: torch.Tensor, out):
    return (qf * scale_b).to(out)


def main():
    g = torch.Generator().manual_seed(20240601)
    bf16, f16, f32 = torch.bfloat16, torch.float16, torch.float32
    arrays: dict[str, np.ndarray] = {}
    manifest: list[dict] = []

    def rnd(*shape, scale=1.0, dtype=bf16):
        return (torch.randn(*shape, generator=g) * scale).to(dtype)

    def student_t3(n):
        z = torch.randn(n, generator=g)
        c = torch.randn(3, n, generator=g)
        return z / torch.sqrt((c * c).sum(0) / 3.0)

    def add(kind, name, x, meta, q, scale, dequant_fn):
        key = f"{kind}:{name}"
        arrays[key + ":x"] = bits(x)
        arrays[key + ":q"] = bits(q)
        arrays[key + ":scale"] = scale.to(f32).reshape(-1).numpy().copy()
        for out in (bf16, f16):
            arrays[key + f":y{CODES[out]}"] = bits(dequant_fn(out))
        manifest.append({"kind": kind, "name": name, "dtype": CODES[x.dtype],
                         "shape": list(x.shape), **meta})

    # ---- FP8 per-tensor (quant_dequant_fp8.py:48-58, reduced sizes) -------
    outlier = torch.full((10_000,), 0.01, dtype=bf16)
    outlier[5000] = 99.5
    fp8_cases = [
        ("toy_1_8", torch.arange(1, 9, dtype=bf16)),
        ("randn3_4096", rnd(4096, scale=3.0)),
        ("single_outlier", outlier),
        ("tail_2049", rnd(2049)),
        ("fp16_parity", rnd(4096, scale=3.0, dtype=f16)),
        ("zeros_eps", torch.zeros(64, dtype=bf16)),
        ("tiny_subnormal", rnd(1000, scale=1e-3)),
        ("mat_37x53", rnd(37, 53, scale=0.5)),
        ("empty", torch.zeros(0, dtype=bf16)),
    ]
    for name, x in fp8_cases:
        q, s = t_quant_fp8(x)
        add("fp8_tensor", name, x, {}, q, s,
            lambda out, q=q, s=s: t_dequant(q.float(), s, out))

    # ---- INT8 per-tensor (quant_dequant_int8.py:134-142) ------------------
    int8_tensor_cases = [
        ("linspace_256", torch.linspace(-1.0, 1.0, 256, dtype=bf16)),
        ("randn3_4096", rnd(4096, scale=3.0)),
        ("single_outlier", outlier),
        ("tail_2049", rnd(2049)),
        ("fp16_parity", rnd(4096, scale=3.0, dtype=f16)),
        ("fp32_input", rnd(3000, scale=2.0, dtype=f32)),
        ("student_t_fp16", (0.5 * student_t3(4096)).to(f16)),
        ("zeros_eps", torch.zeros(64, dtype=f16)),
        ("empty", torch.zeros(0, dtype=f16)),
    ]
    for name, x in int8_tensor_cases:
        q, s = t_quant_int8_tensor(x)
        add("int8_tensor", name, x, {}, q, s,
            lambda out, q=q, s=s: t_dequant(q.float(), s, out))

    # ---- INT8 per-channel (quant_dequant_int8.py:154-158) -----------------
    w_out = rnd(48, 256, scale=0.02)
    w_out[:, [3, 77, 200]] *= 20
    channel_cases = [
        ("w_8x1024", rnd(8, 1024), 0),
        ("w_32x256", rnd(32, 256), 0),
        ("w_outlier_cols_48x256", w_out, 0),
        ("w_outlier_cols_48x256_ax1", w_out, 1),
        ("w_fp32_16x64", rnd(16, 64, dtype=f32), 0),
        ("w_fp16_24x40_ax1", rnd(24, 40, dtype=f16), 1),
        ("odd_5x13", rnd(5, 13), 0),
        ("odd_5x13_ax1", rnd(5, 13), 1),
        ("nd_4x6x10", rnd(4, 6, 10), 0),
        ("row_zero_3x16", torch.cat([torch.zeros(1, 16, dtype=bf16), rnd(2, 16)]), 0),
    ]
    for name, x, axis in channel_cases:
        q, s = t_quant_int8_channel(x, axis)
        rows = x.shape[0]
        qf = q.float().reshape(rows, -1)
        sb = s[:, None] if axis == 0 else s[None, :]
        add("int8_channel", name, x, {"axis": axis}, q, s,
            lambda out, qf=qf, sb=sb, shp=x.shape: t_dequant(qf, sb, out).reshape(shp))

    # ---- INT8 per-group (quant_dequant_int8.py:170-174), grouped 2-D view --
    rowfac = 0.1 + 9.9 * torch.rand(32, 1, generator=g)
    group_cases = [
        ("vec_1024_g32", rnd(1024), 32),
        ("mat_16x1024_g128", rnd(16, 1024), 128),
        ("rowscaled_32x512_g128", (torch.randn(32, 512, generator=g) * rowfac).to(bf16), 128),
        ("mat_32x256_g32", rnd(32, 256), 32),
        ("fp16_16x256_g64", rnd(16, 256, dtype=f16), 64),
        ("fp32_8x96_g96", rnd(8, 96, dtype=f32), 96),
        ("g4096_2x4096", rnd(2, 4096), 4096),
        ("g1_vec_50", rnd(50), 1),
        ("g7_3x21", rnd(3, 21), 7),
        ("g40_5x40", rnd(5, 40), 40),
    ]
    for name, x, gs in group_cases:
        q, s = t_quant_int8_group(x, gs)
        qf = q.float().reshape(-1, gs)
        add("int8_group", name, x, {"group_size": gs}, q, s,
            lambda out, qf=qf, s=s, shp=x.shape: t_dequant(qf, s[:, None], out).reshape(shp))

    # ---- W8A16 (linear.py:97-135), exact float64 accumulation -------------
    for name, (M, K, N, dt, with_bias, oc) in {
        "w8a16_f16_4x64x48": (4, 64, 48, f16, False, []),
        "w8a16_f16_bias_7x96x40": (7, 96, 40, f16, True, []),
        "w8a16_bf16_5x128x64": (5, 128, 64, bf16, True, []),
        "w8a16_f16_outliers_6x64x32": (6, 64, 32, f16, True, [2, 17, 40]),
    }.items():
        x = torch.randn(M, K, generator=g).to(dt)
        w = (0.02 * torch.randn(N, K, generator=g))
        normal = [k for k in range(K) if k not in oc]
        for k in oc:
            x[:, k] = 10.0
        wn = w[:, normal]
        qn, sn = t_quant_int8_channel(wn, 0)
        scales = sn.to(dt)
        bias = (0.1 * torch.randn(N, generator=g)).to(dt) if with_bias else None
        w_out = w[:, oc].to(dt) if oc else None
        x64 = x.double()
        y = (x64[:, normal] @ qn.double().t()) * scales.double()
        if oc:
            y = y + x64[:, oc] @ w_out.double().t()
        if bias is not None:
            y = y + bias.double()
        key = f"w8a16:{name}"
        arrays[key + ":x"] = bits(x)
        arrays[key + ":wq"] = qn.numpy().copy()
        arrays[key + ":scales"] = bits(scales)
        if bias is not None:
            arrays[key + ":bias"] = bits(bias)
        if oc:
            arrays[key + ":outlier_cols"] = np.array(oc, np.int64)
            arrays[key + ":normal_cols"] = np.array(normal, np.int64)
            arrays[key + ":w_out"] = bits(w_out)
        arrays[key + ":y"] = y.float().numpy()
        manifest.append({"kind": "w8a16", "name": name, "dtype": CODES[dt],
                         "shape": [M, K, N], "bias": with_bias, "n_out": len(oc)})

    arrays["manifest"] = np.frombuffer(json.dumps(manifest).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(manifest)} cases)")


if __name__ == "__main__":
    main()
