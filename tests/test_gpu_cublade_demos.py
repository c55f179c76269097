"""The reference's own usage, through the reference's import name.

Imports the library only as ``cublade.*`` (the way the reference's examples
do: ``from cublade.quantization import dequantize_tensor, quantize_tensor``,
examples/quantization/quant_dequant_fp8.py:14, quant_dequant_int8.py:13,
w8a16_toy_model.py:17) and runs the case lists of those demos:

* quant_dequant_fp8.py:48-58   per-tensor FP8 round trips (6 cases)
* quant_dequant_int8.py:51-91  per-tensor (6), per-channel (3) and per-group
                               (3) INT8 round trips
* w8a16_toy_model.py:23-89     quantize_model on the 3-layer MLP, run as the
                               demo does (CPU model and input) and on the GPU

The demos only print error tables; here every code, scale and dequantized
value is compared bit for bit with the CPU oracle on the same input, and the
W8A16 outputs within rtol = atol = 1e-2 of the oracle's exact accumulation.
Inputs are drawn as the demos draw them (global seed, on the device).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from tests._util import (CODE_OF, assert_array_equal, assert_bits_equal_16, assert_fp8_equal,
                         bits)

pytestmark = pytest.mark.gpu

DEVICE = "cuda"
TOL = dict(rtol=1e-2, atol=1e-2)


def _fp8_cases():
    """quant_dequant_fp8.py:44-58."""
    torch.manual_seed(0)
    bf16 = torch.bfloat16
    cases = [
        ("toy [1..8]", torch.arange(1, 9, dtype=bf16, device=DEVICE)),
        ("1M random", torch.randn(1_000_000, dtype=bf16, device=DEVICE) * 3.0),
        ("16M random", torch.randn(16_000_000, dtype=bf16, device=DEVICE) * 3.0),
        ("single outlier", torch.full((10_000,), 0.01, dtype=bf16, device=DEVICE)),
        ("2049 (tail path)", torch.randn(2049, dtype=bf16, device=DEVICE)),
        ("fp16 parity", torch.randn(1_000_000, dtype=torch.float16, device=DEVICE) * 3.0),
    ]
    cases[3][1][5000] = 99.5
    return cases


def _int8_cases():
    """quant_dequant_int8.py:44-91: (name, x, mode, kwargs)."""
    torch.manual_seed(0)
    bf16 = torch.bfloat16
    pt = [
        ("toy [-1..1]/255", torch.linspace(-1.0, 1.0, 256, dtype=bf16, device=DEVICE)),
        ("1M random N(0,3)", torch.randn(1_000_000, dtype=bf16, device=DEVICE) * 3.0),
        ("16M random", torch.randn(16_000_000, dtype=bf16, device=DEVICE) * 3.0),
        ("single outlier", torch.full((10_000,), 0.01, dtype=bf16, device=DEVICE)),
        ("2049 (tail path)", torch.randn(2049, dtype=bf16, device=DEVICE)),
        ("fp16 parity", torch.randn(1_000_000, dtype=torch.float16, device=DEVICE) * 3.0),
    ]
    pt[3][1][5000] = 99.5
    pc = [
        ("8x1024 weight", torch.randn(8, 1024, dtype=bf16, device=DEVICE)),
        ("1024x1024 weight", torch.randn(1024, 1024, dtype=bf16, device=DEVICE)),
        ("4096x4096 weight", torch.randn(4096, 4096, dtype=bf16, device=DEVICE)),
    ]
    pg = [
        ("1024-vec G=32", torch.randn(1024, dtype=bf16, device=DEVICE),
         {"group_size": 32, "ch_axis": 0}),
        ("1024x1024 G=128 ax-1", torch.randn(1024, 1024, dtype=bf16, device=DEVICE),
         {"group_size": 128, "ch_axis": -1}),
        ("4096x4096 G=32 ax-1", torch.randn(4096, 4096, dtype=bf16, device=DEVICE),
         {"group_size": 32, "ch_axis": -1}),
    ]
    return ([(n, x, "tensor", {}) for n, x in pt]
            + [(n, x, "channel", {"ch_axis": 0}) for n, x in pc]
            + [(n, x, "group", kw) for n, x, kw in pg])


def test_reference_import_lines():
    """The import lines of the reference's examples and bindings resolve, and
    name the same objects as the implementation package."""
    import cublade
    import cublade_amd
    from cublade import _loader
    from cublade._loader import CSRC, is_loaded, load_cuda_module, load_error  # noqa: F401
    from cublade.bindings.cuda import dequantize_fp8, dequantize_int8, quantize_fp8, quantize_int8
    from cublade.quantization import (QuantizedTensor, cuBladeW8A16LinearLayer,  # noqa: F401
                                      dequantize_tensor, quantize_model, quantize_tensor)
    assert quantize_tensor is cublade_amd.quantization.quantize_tensor
    assert cublade.quantize_tensor is quantize_tensor
    assert _loader is cublade_amd._loader
    assert callable(quantize_fp8.quantize_per_tensor_fp8)
    assert callable(dequantize_fp8.dequantize_per_tensor_fp8)
    for f in ("quantize_per_tensor_int8", "quantize_per_channel_int8", "quantize_per_group_int8"):
        assert callable(getattr(quantize_int8, f))
    for f in ("dequantize_per_tensor_int8", "dequantize_per_channel_int8",
              "dequantize_per_group_int8"):
        assert callable(getattr(dequantize_int8, f))


@pytest.mark.parametrize("idx", range(6))
def test_fp8_demo_cases(idx):
    from cublade.quantization import dequantize_tensor, quantize_tensor
    name, x = _fp8_cases()[idx]
    print(f"[fp8 demo] {name} shape={tuple(x.shape)} dtype={x.dtype}", flush=True)
    qt = quantize_tensor(x.contiguous(), dtype=torch.float8_e4m3fn, mode="tensor")
    y = dequantize_tensor(qt)
    code = CODE_OF[x.dtype]
    xb = bits(x)
    qo, so = oracle.quant_fp8_tensor(xb, code)
    assert_fp8_equal(bits(qt.data), qo, f"{name} q")
    assert_array_equal(bits(qt.scale).reshape(-1).view(np.uint32),
                       np.array([so], np.float32).view(np.uint32), f"{name} scale")
    assert y.dtype == x.dtype and y.shape == x.shape
    assert_bits_equal_16(bits(y), oracle.dequant_fp8_tensor(qo, so, code), code, f"{name} y")
    if name == "toy [1..8]":
        # the values the demo prints (quant_dequant_fp8.py:71-79)
        assert [f"0x{b:02x}" for b in bits(qt.data).tolist()] == [
            "0x66", "0x6e", "0x72", "0x76", "0x79", "0x7a", "0x7c", "0x7e"]
        assert y.float().tolist() == [1.0, 2.0, 2.859375, 4.0, 5.15625, 5.71875, 6.84375, 8.0]


@pytest.mark.parametrize("idx", range(12))
def test_int8_demo_cases(idx):
    from cublade.quantization import dequantize_tensor, quantize_tensor
    name, x, mode, kw = _int8_cases()[idx]
    print(f"[int8 demo] {name} mode={mode} shape={tuple(x.shape)}", flush=True)
    qt = quantize_tensor(x.contiguous(), dtype=torch.int8, mode=mode, **kw)
    y = dequantize_tensor(qt)
    code = CODE_OF[x.dtype]
    xb = bits(x)
    if mode == "tensor":
        qo, so = oracle.quant_int8_tensor(xb, code)
        yo = oracle.dequant_int8_tensor(qo, so, code)
        so = np.array([so], np.float32)
    elif mode == "channel":
        qo, so = oracle.quant_int8_channel(xb, code, axis=0)
        yo = oracle.dequant_int8_channel(qo, so, code, axis=0)
    else:
        G = kw["group_size"]
        qo, so = oracle.quant_int8_group(xb.reshape(-1, G), code, G)
        yo = oracle.dequant_int8_group(qo, so, G, code)
    assert_array_equal(bits(qt.data), qo, f"{name} q")
    assert_array_equal(bits(qt.scale).reshape(-1).view(np.uint32),
                       np.asarray(so, np.float32).view(np.uint32), f"{name} scale")
    assert y.dtype == x.dtype and y.shape == x.shape
    assert_bits_equal_16(bits(y), yo, code, f"{name} y")
    if name == "toy [-1..1]/255":
        q = bits(qt.data)
        assert q[:10].tolist() == list(range(-127, -117))
        assert q[123:133].tolist() == [-4, -3, -2, -1, 0, 0, 1, 2, 3, 4]


class DummyModel(nn.Module):
    """w8a16_toy_model.py:23-35."""

    def __init__(self):
        super().__init__()
        self.fc1 = nn.Linear(128, 256)
        self.fc2 = nn.Linear(256, 128)
        self.fc3 = nn.Linear(128, 10)

    def forward(self, x):
        x = torch.relu(self.fc1(x))
        x = torch.relu(self.fc2(x))
        return self.fc3(x)


def _check_layer(layer, w_fp32, x, y):
    """Codes and scales vs the oracle's channel quant of the fp32 weight, and
    the layer output vs the oracle's W8A16 on the same input."""
    qo, so = oracle.quant_int8_channel(w_fp32.detach().cpu().numpy(), oracle.F32, axis=0)
    assert_array_equal(bits(layer.int8_weights), qo, "int8_weights")
    assert_array_equal(bits(layer.scales).view(np.uint32), so.view(np.uint32), "scales")
    ref = oracle.w8a16_linear(bits(x), oracle.F32, qo, so,
                              bias=bits(layer.bias.detach()))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, **TOL)


@pytest.mark.parametrize("where", ["cpu-model (as the demo)", "gpu-model"])
def test_w8a16_toy_model(where):
    from cublade.quantization import cuBladeW8A16LinearLayer, quantize_model
    print(f"[w8a16 toy] {where}", flush=True)
    torch.manual_seed(42)
    model_fp = DummyModel().eval()
    model_w8 = DummyModel().eval()
    model_w8.load_state_dict(model_fp.state_dict())
    dev = "cpu" if where.startswith("cpu") else DEVICE
    model_fp = model_fp.to(dev)
    model_w8 = model_w8.to(dev)
    weights = {n: getattr(model_w8, n).weight.detach().clone() for n in ("fc1", "fc2", "fc3")}
    model_w8 = quantize_model(model_w8, quant_type="w8a16", inplace=True)
    for n in ("fc1", "fc2", "fc3"):
        layer = getattr(model_w8, n)
        assert isinstance(layer, cuBladeW8A16LinearLayer)
        assert layer.int8_weights.dtype == torch.int8 and layer.int8_weights.device.type == dev
    x = torch.randn(4, 128).to(dev)
    with torch.no_grad():
        out_fp = model_fp(x)
        out_w8 = model_w8(x)
        h1 = torch.relu(model_w8.fc1(x))
        h2 = torch.relu(model_w8.fc2(h1))
        _check_layer(model_w8.fc1, weights["fc1"], x, model_w8.fc1(x))
        _check_layer(model_w8.fc2, weights["fc2"], h1, model_w8.fc2(h1))
        _check_layer(model_w8.fc3, weights["fc3"], h2, model_w8.fc3(h2))
    # the demo's own "Good" thresholds (w8a16_toy_model.py:83-84)
    mse = (out_fp - out_w8).pow(2).mean().item()
    max_err = (out_fp - out_w8).abs().max().item()
    assert mse < 0.01 and max_err < 0.5, (mse, max_err)
