"""Pin the oracle's quant / dequant / W8A16 entry points (CPU only).

Checks, independent of oracle/cbq_oracle.c:
* the committed golden vectors (torch-CPU restatement, tests/golden/);
* closed-form known answers for the reference demos' toy cases
  (examples/quantization/quant_dequant_fp8.py:49,71-79 and
  examples/quantization/quant_dequant_int8.py:135,188-196);
* invariants fixed by the mathematics (transpose, group/channel/tensor
  equivalences, range and round-trip error bounds).
"""
import numpy as np
import pytest
import torch

import oracle
from tests import _golden as G
from tests._util import assert_bits_equal_16, bits


def _y_key(out_code):
    return f"y{out_code}"


@pytest.mark.parametrize("meta,arr", G.cases("fp8_tensor"), ids=G.ids("fp8_tensor"))
def test_fp8_tensor_golden(meta, arr):
    x = arr["x"].reshape(meta["shape"])
    q, s = oracle.quant_fp8_tensor(x, meta["dtype"])
    assert np.array_equal(q.reshape(-1), arr["q"].reshape(-1))
    assert np.float32(s).view(np.uint32) == arr["scale"][0].view(np.uint32)
    for out in (oracle.F16, oracle.BF16):
        y = oracle.dequant_fp8_tensor(q, s, out)
        assert np.array_equal(y.reshape(-1), arr[_y_key(out)].reshape(-1))


@pytest.mark.parametrize("meta,arr", G.cases("int8_tensor"), ids=G.ids("int8_tensor"))
def test_int8_tensor_golden(meta, arr):
    x = arr["x"].reshape(meta["shape"])
    q, s = oracle.quant_int8_tensor(x, meta["dtype"])
    assert np.array_equal(q.reshape(-1), arr["q"].reshape(-1))
    assert np.float32(s).view(np.uint32) == arr["scale"][0].view(np.uint32)
    for out in (oracle.F16, oracle.BF16):
        y = oracle.dequant_int8_tensor(q, s, out)
        assert np.array_equal(y.reshape(-1), arr[_y_key(out)].reshape(-1))


@pytest.mark.parametrize("meta,arr", G.cases("int8_channel"), ids=G.ids("int8_channel"))
def test_int8_channel_golden(meta, arr):
    x = arr["x"].reshape(meta["shape"])
    q, s = oracle.quant_int8_channel(x, meta["dtype"], axis=meta["axis"])
    assert np.array_equal(q.reshape(-1), arr["q"].reshape(-1))
    assert np.array_equal(s.view(np.uint32), arr["scale"].view(np.uint32))
    for out in (oracle.F16, oracle.BF16):
        y = oracle.dequant_int8_channel(q, s, out, axis=meta["axis"])
        assert np.array_equal(y.reshape(-1), arr[_y_key(out)].reshape(-1))


@pytest.mark.parametrize("meta,arr", G.cases("int8_group"), ids=G.ids("int8_group"))
def test_int8_group_golden(meta, arr):
    x = arr["x"].reshape(meta["shape"])
    gs = meta["group_size"]
    q, s = oracle.quant_int8_group(x, meta["dtype"], gs)
    assert np.array_equal(q.reshape(-1), arr["q"].reshape(-1))
    assert np.array_equal(s.view(np.uint32), arr["scale"].view(np.uint32))
    for out in (oracle.F16, oracle.BF16):
        y = oracle.dequant_int8_group(q, s, gs, out)
        assert np.array_equal(y.reshape(-1), arr[_y_key(out)].reshape(-1))


@pytest.mark.parametrize("meta,arr", G.cases("w8a16"), ids=G.ids("w8a16"))
def test_w8a16_golden(meta, arr):
    M, K, N = meta["shape"]
    x = arr["x"].reshape(M, K)
    y = oracle.w8a16_linear(x, meta["dtype"], arr["wq"], arr["scales"], bias=arr.get("bias"),
                            normal_cols=arr.get("normal_cols"),
                            outlier_cols=arr.get("outlier_cols"), w_out=arr.get("w_out"))
    np.testing.assert_allclose(y, arr["y"], rtol=1e-6, atol=1e-6)
    # row subset is the same computation restricted to those rows
    rows = np.array([M - 1, 0], np.int64)
    ys = oracle.w8a16_linear(x, meta["dtype"], arr["wq"], arr["scales"], bias=arr.get("bias"),
                             normal_cols=arr.get("normal_cols"),
                             outlier_cols=arr.get("outlier_cols"), w_out=arr.get("w_out"),
                             rows=rows)
    assert np.array_equal(ys, y[rows])


def _bf16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_fp8_toy_known_answer():
    """x = bf16 [1..8]: inv = 56, scale = 0x3c924925; 168 -> 160 and 336 -> 320
    are ties to even (quant_dequant_fp8.py:49 toy case)."""
    q, s = oracle.quant_fp8_tensor(_bf16(torch.arange(1, 9, dtype=torch.bfloat16)), oracle.BF16)
    assert list(q) == [0x66, 0x6E, 0x72, 0x76, 0x79, 0x7A, 0x7C, 0x7E]
    assert np.float32(s).view(np.uint32) == 0x3C924925
    y = oracle.dequant_fp8_tensor(q, s, oracle.BF16)
    assert list(y) == [0x3F80, 0x4000, 0x4037, 0x4080, 0x40A5, 0x40B7, 0x40DB, 0x4100]


def test_int8_linspace_known_answer():
    """linspace(-1, 1, 256) bf16 (quant_dequant_int8.py:135): inv = 127."""
    x = _bf16(torch.linspace(-1.0, 1.0, 256, dtype=torch.bfloat16))
    q, s = oracle.quant_int8_tensor(x, oracle.BF16)
    assert np.float32(s) == np.float32(1.0) / np.float32(127.0)
    assert list(q[:10]) == list(range(-127, -117))
    assert list(q[123:133]) == [-4, -3, -2, -1, 0, 0, 1, 2, 3, 4]


def test_eps_floor_and_empty():
    q, s = oracle.quant_int8_tensor(np.zeros(16, np.float32), oracle.F32)
    assert np.all(q == 0) and np.float32(s) == np.float32(1.0) / (np.float32(127.0) / np.float32(1e-12))
    q, s = oracle.quant_fp8_tensor(np.zeros(0, np.uint16), oracle.BF16)
    assert q.size == 0 and s == 0.0


def _rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return _bf16((torch.randn(*shape, generator=g) * scale).to(torch.bfloat16))


def test_channel_axis1_is_axis0_of_transpose():
    x = _rand_bf16((37, 29), 1)
    q1, s1 = oracle.quant_int8_channel(x, oracle.BF16, axis=1)
    q0, s0 = oracle.quant_int8_channel(np.ascontiguousarray(x.T), oracle.BF16, axis=0)
    assert np.array_equal(q1, q0.T) and np.array_equal(s1, s0)
    y1 = oracle.dequant_int8_channel(q1, s1, oracle.BF16, axis=1)
    y0 = oracle.dequant_int8_channel(q0, s0, oracle.BF16, axis=0)
    assert np.array_equal(y1, y0.T)


def test_group_equivalences():
    x = _rand_bf16((12, 64), 2)
    qg, sg = oracle.quant_int8_group(x, oracle.BF16, 64)
    qc, sc = oracle.quant_int8_channel(x, oracle.BF16, axis=0)
    assert np.array_equal(qg, qc) and np.array_equal(sg, sc)
    q1, s1 = oracle.quant_int8_group(x, oracle.BF16, x.size)
    qt, st = oracle.quant_int8_tensor(x, oracle.BF16)
    assert np.array_equal(q1, qt) and s1[0] == st


def test_range_and_round_trip_bound():
    x = _rand_bf16((4096,), 3, scale=5.0)
    xf = oracle.to_f32(x, oracle.BF16)
    q, s = oracle.quant_int8_tensor(x, oracle.BF16)
    assert np.abs(q).max() == 127 and q.min() >= -127
    yf = np.float32(s) * q.astype(np.float32)
    assert np.all(np.abs(yf - xf) <= np.float32(s) * 0.5 * (1 + 1e-5))
    q8, s8 = oracle.quant_fp8_tensor(x, oracle.BF16)
    v = oracle.decode_e4m3(q8)
    assert np.abs(v).max() == 448.0


def test_w8a16_matches_numpy_float64():
    g = torch.Generator().manual_seed(9)
    M, K, N = 3, 40, 24
    x = torch.randn(M, K, generator=g).to(torch.float16)
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 0.01).to(torch.float16)
    b = torch.randn(N, generator=g).to(torch.float16)
    y = oracle.w8a16_linear(_bf16(x), oracle.F16, wq.numpy(), _bf16(s), bias=_bf16(b))
    ref = (x.double().numpy() @ wq.double().numpy().T) * s.double().numpy() + b.double().numpy()
    np.testing.assert_allclose(y, ref.astype(np.float32), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("qd", [torch.int8, torch.float8_e4m3fn])
def test_torch_cpu_restatement_matches_c_oracle(dt, qd):
    """oracle/torch_cpu.py (the CPU baseline of bench.py) gives the C
    oracle's codes, scale and dequantized values bit for bit, NaN / inf /
    -0 / tiny inputs included."""
    from oracle import torch_cpu
    if qd == torch.float8_e4m3fn and dt == torch.float32:
        pytest.skip("FP8 takes fp16 / bf16 inputs only")
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(50_003, generator=g) * 3).to(dt)
    x[5] = float("nan")
    x[7] = 60000.0 if dt == torch.float16 else float("inf")
    x[9] = -0.0
    x[11] = 1e-30 if dt != torch.float16 else 1e-7
    code = {torch.float16: oracle.F16, torch.bfloat16: oracle.BF16, torch.float32: oracle.F32}[dt]
    q, s = torch_cpu.quant_tensor(x, qd)
    if qd == torch.int8:
        qo, so = oracle.quant_int8_tensor(bits(x), code)
    else:
        qo, so = oracle.quant_fp8_tensor(bits(x), code)
    assert np.array_equal(bits(q).view(np.uint8), qo.view(np.uint8))
    assert np.float32(s.item()).view(np.uint32) == np.float32(so).view(np.uint32)
    out = torch.bfloat16 if dt == torch.float32 else dt
    y = torch_cpu.dequant_tensor(q, s, out)
    oc = oracle.BF16 if out == torch.bfloat16 else oracle.F16
    yo = (oracle.dequant_int8_tensor(qo, so, oc) if qd == torch.int8
          else oracle.dequant_fp8_tensor(qo, so, oc))
    assert_bits_equal_16(bits(y), yo, oc, "dequant")   # any NaN matches any NaN
