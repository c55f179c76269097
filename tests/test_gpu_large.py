"""Maximum sizes: every quant / dequant mode and the W8A16 linear on tensors
of more than 2^31 elements (64-bit element offsets in every kernel that
indexes them).

The oracle cannot run at these sizes, so the inputs are built from few
distinct values: constant rows, columns or groups plus a few spikes placed
past element 2^31. A row (column, group) of identical values with the same
maximum quantizes like a short proxy row holding those values, so the
expected codes, scales and dequantized values come from the oracle on the
proxies; the full tensors are then compared on the GPU (bit patterns,
exact). The W8A16 case checks sampled rows against the oracle.
"""
from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

import oracle
from tests._util import bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
BIG = (1 << 31) + 77


@pytest.fixture(autouse=True)
def _free():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def h(v: float) -> np.ndarray:
    """fp16 bit pattern of v."""
    return np.array([v], np.float16).view(np.uint16)


def f16_bits(values) -> np.ndarray:
    return np.asarray(values, np.float16).view(np.uint16)


def u16(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


def chan(x2: np.ndarray, axis: int):
    """Oracle channel quant of a small proxy: (codes [rows, cols], scales)."""
    qo, so = oracle.quant_int8_channel(x2, oracle.F16, axis=axis)
    return np.asarray(qo).reshape(x2.shape), np.asarray(so, np.float32).reshape(-1)


def deq_chan(q2: np.ndarray, s: np.ndarray, axis: int) -> np.ndarray:
    """Oracle channel dequant of a proxy, fp16 bits as int16, flattened."""
    y = oracle.dequant_int8_channel(q2, s, oracle.F16, axis=axis)
    return np.asarray(y, np.uint16).reshape(-1).view(np.int16)


def expect_all(t: torch.Tensor, value: int, except_at=(), what=""):
    """Every element of t equals `value` except at the listed flat indices."""
    flat = t.reshape(-1)
    bad = int((flat != value).sum().item())
    assert bad == len(except_at), f"{what}: {bad} elements differ from {value}"
    for i in except_at:
        assert int(flat[i].item()) != value, f"{what}: spike at {i} lost"


@pytest.mark.parametrize("fp8", [False, True])
def test_tensor_past_2g(fp8):
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    print(f"[large] per-tensor fp8={fp8} n={BIG}", flush=True)
    c, s1, s2 = 0.3, 7.0, -9.5
    p1, p2 = 5, (1 << 31) + 40
    x = torch.full((BIG,), c, dtype=torch.float16, device=DEV)
    x[p1], x[p2] = s1, s2
    proxy = f16_bits([c, s1, s2])
    if fp8:
        qt = quantize_tensor(x, dtype=torch.float8_e4m3fn, mode="tensor")
        qo, so = oracle.quant_fp8_tensor(proxy, oracle.F16)
        yo = oracle.dequant_fp8_tensor(qo, so, oracle.F16)
        q = qt.data.view(torch.uint8)
    else:
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        qo, so = oracle.quant_int8_tensor(proxy, oracle.F16)
        yo = oracle.dequant_int8_tensor(qo, so, oracle.F16)
        q = qt.data
    del x
    assert bits(qt.scale).reshape(-1).view(np.uint32)[0] == np.float32(so).view(np.uint32)
    qo = np.asarray(qo).reshape(-1).astype(np.int64)
    expect_all(q, int(qo[0]), (p1, p2), "codes")
    assert int(q[p1].item()) == int(qo[1]) and int(q[p2].item()) == int(qo[2])
    y = dequantize_tensor(qt)
    del qt, q
    yo = np.asarray(yo, np.uint16).reshape(-1).view(np.int16).astype(np.int64)
    expect_all(u16(y), int(yo[0]), (p1, p2), "y")
    assert int(u16(y)[p1].item()) == int(yo[1]) and int(u16(y)[p2].item()) == int(yo[2])


def test_channel_axis0_past_2g():
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    R, C = (1 << 18) + 3, 8192
    print(f"[large] channel axis 0 {R}x{C}", flush=True)
    vals = [0.01 * (k + 1) for k in range(7)]
    x = torch.tensor(vals, dtype=torch.float16, device=DEV)[torch.arange(R, device=DEV) % 7]
    x = x[:, None].expand(R, C).contiguous()
    spikes = [(R // 2, 5, -2.0), (R - 1, C - 1, 3.0)]
    for r, col, v in spikes:
        x[r, col] = v
    qt = quantize_tensor(x, dtype=torch.int8, mode="channel", ch_axis=0)
    del x
    # expected per row: constant rows quantize like [c]; spike rows like [c, spike]
    s_exp = np.empty(R, np.float32)
    q_row = np.empty(R, np.int64)
    for k, v in enumerate(vals):
        qo, so = chan(f16_bits([v]).reshape(1, 1), 0)
        s_exp[k::7] = so[0]
        q_row[k::7] = qo[0, 0]
    spike_q = {}
    for r, col, v in spikes:
        qo, so = chan(f16_bits([vals[r % 7], v]).reshape(1, 2), 0)
        s_exp[r] = so[0]
        q_row[r] = qo[0, 0]
        spike_q[(r, col)] = int(qo[0, 1])
    assert np.array_equal(bits(qt.scale).view(np.uint32), s_exp.view(np.uint32))
    qe = torch.from_numpy(q_row.astype(np.int8)).to(DEV)
    bad = qt.data != qe[:, None]
    assert int(bad.sum().item()) == len(spikes)
    for (r, col), qv in spike_q.items():
        assert int(qt.data[r, col].item()) == qv
    del bad
    y = dequantize_tensor(qt)
    y_row = np.empty(R, np.int16)
    for k in range(7):
        y_row[k::7] = deq_chan(np.array([[q_row[k]]], np.int8), s_exp[k:k + 1], 0)[0]
    for r, col, _ in spikes:
        yo = deq_chan(np.array([[q_row[r], spike_q[(r, col)]]], np.int8), s_exp[r:r + 1], 0)
        y_row[r] = yo[0]
        assert int(u16(y)[r, col].item()) == int(yo[1])
    ye = torch.from_numpy(y_row).to(DEV)
    assert int((u16(y) != ye[:, None]).sum().item()) == len(spikes)


def test_channel_axis1_and_group_past_2g():
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    R, C = (1 << 18) + 3, 8192
    print(f"[large] channel axis 1 / group {R}x{C}", flush=True)
    vals = [0.02 * ((k % 5) + 1) for k in range(C)]
    col_v = torch.tensor(vals, dtype=torch.float16, device=DEV)
    x = col_v[None, :].expand(R, C).contiguous()
    r_sp, c_sp, v_sp = R - 1, 7, 5.0                 # past element 2^31
    x[r_sp, c_sp] = v_sp
    # per column: constant columns quantize like [v]; column 7 like [v, spike]
    qt = quantize_tensor(x, dtype=torch.int8, mode="channel", ch_axis=1)
    s_exp = np.empty(C, np.float32)
    q_col = np.empty(C, np.int64)
    for k in range(5):
        qo, so = chan(f16_bits([vals[k]]).reshape(1, 1), 1)
        s_exp[k::5] = so[0]
        q_col[k::5] = qo[0, 0]
    qo, so = chan(f16_bits([vals[c_sp], v_sp]).reshape(2, 1), 1)
    s_exp[c_sp], q_col[c_sp], q_spike = so[0], qo[0, 0], int(qo[1, 0])
    assert np.array_equal(bits(qt.scale).view(np.uint32), s_exp.view(np.uint32))
    qe = torch.from_numpy(q_col.astype(np.int8)).to(DEV)
    assert int((qt.data != qe[None, :]).sum().item()) == 1
    assert int(qt.data[r_sp, c_sp].item()) == q_spike
    y = dequantize_tensor(qt)
    y_col = deq_chan(q_col.astype(np.int8).reshape(1, C), s_exp, 1)
    ye = torch.from_numpy(y_col).to(DEV)
    assert int((u16(y) != ye[None, :]).sum().item()) == 1
    del qt, y
    # groups of 128 along the last axis: each group holds 5-periodic column
    # values, so every group quantizes like the proxy of its 128 values
    G = 128
    qt = quantize_tensor(x, dtype=torch.int8, mode="group", group_size=G, ch_axis=-1)
    del x
    ng = R * C // G
    proxy = np.stack([f16_bits(vals[g * G:(g + 1) * G]) for g in range(C // G)])
    qo, so = oracle.quant_int8_group(proxy, oracle.F16, G)
    qo = np.asarray(qo, np.int8).reshape(C // G, G)
    spike_row = f16_bits(vals[0:G]).copy()
    spike_row[c_sp] = h(v_sp)[0]
    qs, ss = oracle.quant_int8_group(spike_row.reshape(1, G), oracle.F16, G)
    qs = np.asarray(qs, np.int8).reshape(-1)
    g_sp = (r_sp * C + c_sp) // G
    s_exp = np.tile(np.asarray(so, np.float32), R)
    s_exp[g_sp] = ss[0]
    assert np.array_equal(bits(qt.scale).view(np.uint32), s_exp.view(np.uint32))
    qe = torch.from_numpy(qo.reshape(-1)).to(DEV)
    bad = qt.data.view(R, C) != qe[None, :]
    assert int(bad.sum().item()) == int((qs != qo[0]).sum())
    assert np.array_equal(qt.data.view(ng, G)[g_sp].cpu().numpy(), qs)
    del bad
    y = dequantize_tensor(qt)
    yo = np.asarray(oracle.dequant_int8_group(qo, np.asarray(so, np.float32), G, oracle.F16),
                    np.uint16).reshape(C // G, G).view(np.int16)
    ys = np.asarray(oracle.dequant_int8_group(qs.reshape(1, G), np.asarray(ss, np.float32), G,
                                              oracle.F16), np.uint16).reshape(-1).view(np.int16)
    assert np.array_equal(u16(y).view(ng, G)[g_sp].cpu().numpy(), ys)
    ye = torch.from_numpy(np.ascontiguousarray(yo.reshape(-1))).to(DEV)
    assert int((u16(y).view(R, C) != ye[None, :]).sum().item()) == int((ys != yo[0]).sum())


def test_w8a16_activations_past_2g():
    """x [2^19 + 5, 4096] fp16 (2^31 + 20480 elements): the tile kernel that
    addresses x with 64-bit offsets; sampled rows against the oracle."""
    from cublade_amd.bindings.hip import w8a16_linear
    M, K, N = (1 << 19) + 5, 4096, 64
    print(f"[large] w8a16 M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(3)
    rows = np.array([0, 1, M // 2, M - 2, M - 1])
    xs = torch.randn(len(rows), K, generator=g).half()
    x = torch.zeros(M, K, dtype=torch.float16, device=DEV)
    x[torch.from_numpy(rows).to(DEV)] = xs.to(DEV)
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int16).to(torch.int8)
    s = (torch.rand(N, generator=g) * 1e-3 + 1e-4).half()
    y = w8a16_linear(x, wq.to(DEV), s.to(DEV))
    del x
    ref = oracle.w8a16_linear(bits(xs), oracle.F16, wq.numpy(), bits(s))
    np.testing.assert_allclose(y[torch.from_numpy(rows).to(DEV)].float().cpu().numpy(), ref,
                               rtol=1e-2, atol=1e-2)
    assert int((y.float().abs().sum(dim=1) != 0).sum().item()) == len(rows)
