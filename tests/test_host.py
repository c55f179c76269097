"""Host-side tests (no GPU): the C-ABI library loads and exports every
declared symbol, its argument validation fails before any device work, the
loader memoises failures, and the Python layer's host logic (checks, outlier
utilities, layer replacement, CPU branch, state_dict layouts) behaves like
the reference's."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from tests._util import bits

ROOT = Path(__file__).resolve().parents[1]


def _lib():
    from cublade_amd import _abi
    return _abi.lib()


def declared_symbols():
    text = (ROOT / "include" / "cublade_quant.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cbq_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib()
    names = declared_symbols()
    assert len(names) == 27
    for n in names:
        assert hasattr(L, n), n
    from cublade_amd import _abi
    assert set(names) == set(_abi.SIGNATURES)


def test_abi_version_and_error_slot():
    L = _lib()
    assert L.cbq_abi_version() == 200
    assert L.cbq_last_error() in (b"",) or isinstance(L.cbq_last_error(), bytes)


def _einval(rc, needle):
    L = _lib()
    assert rc == 1
    assert needle in L.cbq_last_error().decode()


def test_abi_rejects_bad_arguments_without_device_work():
    L = _lib()
    P = ctypes.c_void_p
    fake = P(0x1000)
    _einval(L.cbq_quant_fp8_tensor(fake, 0, 16, 1e-12, fake, 256, fake, fake, None), "dtype")
    # the allocation-free variant checks its arguments before any device call
    _einval(L.cbq_quant_fp8_tensor_noalloc(fake, 0, 16, 1e-12, fake, fake, None), "dtype")
    _einval(L.cbq_quant_fp8_tensor_noalloc(None, 2, 16, 1e-12, fake, fake, None), "null")
    _einval(L.cbq_quant_fp8_tensor_noalloc(fake, 2, -1, 1e-12, fake, fake, None), "negative")
    assert L.cbq_quant_fp8_tensor_noalloc(None, 2, 0, 1e-12, None, None, None) == 0
    _einval(L.cbq_quant_int8_tensor(fake, 1, 16, 1e-12, fake, 1024, fake, fake, None), "workspace")
    _einval(L.cbq_quant_int8_group(fake, 2, 4, 0, 1e-12, fake, fake, None), "group_size")
    _einval(L.cbq_quant_int8_group(fake, 2, 4, 4097, 1e-12, fake, fake, None), "group_size")
    _einval(L.cbq_quant_int8_channel(fake, 2, 4, 4, 2, 1e-12, fake, 256, fake, fake, None), "axis")
    _einval(L.cbq_quant_int8_channel(fake, 2, 64, 64, 1, 1e-12, fake, 256, fake, fake, None),
            "workspace")
    _einval(L.cbq_dequant_fp8_tensor(fake, fake, 16, fake, 0, None), "out_dtype")
    _einval(L.cbq_dequant_int8_group(fake, fake, 4, 8, fake, 3, None), "out_dtype")
    _einval(L.cbq_dequant_int8_channel(fake, fake, 4, 8, 5, fake, 1, None), "axis")
    _einval(L.cbq_w8a16_linear(fake, 7, fake, fake, None, None, 0, None, 4, 4, 4, fake, 256,
                               fake, None), "activation dtype")
    _einval(L.cbq_w8a16_linear(fake, 1, fake, fake, None, None, 2, None, 4, 4, 4, fake, 256,
                               fake, None), "outlier")
    _einval(L.cbq_quant_int8_tensor(None, 1, 16, 1e-12, fake, 256, fake, fake, None), "null")
    # empty inputs are a successful no-op (nothing is dereferenced)
    assert L.cbq_quant_fp8_tensor(None, 1, 0, 1e-12, None, 0, None, None, None) == 0
    assert L.cbq_quant_int8_group(None, 1, 0, 32, 1e-12, None, None, None) == 0
    assert L.cbq_w8a16_linear(None, 1, None, None, None, None, 0, None, 0, 8, 8, None, 0,
                              None, None) == 0


def test_workspace_sizes():
    L = _lib()
    from cublade_amd import _abi
    C = _abi.WS_CTRL_BYTES
    assert L.cbq_quant_int8_channel_ws_bytes(100, 100, 0) == C
    # few long rows on axis 0: one partial maximum per slice of each row (no
    # device here: 256 CUs assumed, 4 workgroups per CU, slices >= 8192
    # elements, at most 256 per row)
    assert L.cbq_quant_int8_channel_ws_bytes(64, 1 << 20, 0) == C + 4 * 64 * 16
    assert L.cbq_quant_int8_channel_ws_bytes(8, 1 << 21, 0) == C + 4 * 8 * 128
    assert L.cbq_quant_int8_channel_ws_bytes(256, 262144, 0) == C + 4 * 256 * 4
    assert L.cbq_quant_int8_channel_ws_bytes(512, 65536, 0) == C     # enough rows
    assert L.cbq_quant_int8_channel_ws_bytes(255, 8200, 0) == C      # rows too short
    assert L.cbq_quant_int8_channel_nd_ws_bytes(1, 4, 65536) == C + 4 * 4 * 8
    assert L.cbq_quant_tensor_ws_bytes() == C + 4 * 2048
    big = L.cbq_quant_int8_channel_ws_bytes(28672, 8192, 1)
    assert big >= C + 8192 * 4 * 2 and big < 64 << 20
    F16, F32 = _abi.F16, _abi.F32
    # M <= 16, fp16: the weight-streaming kernel, no partials. fp32 activations:
    # the larger of the two-plane path's needs (two bf16 planes of x, then 2
    # planes x 2 k-ranges x 43 tiles of 128 x 256 fp32 partials) and the
    # general kernel's (16 k-ranges of [16, 11008] fp32 partial sums)
    assert L.cbq_w8a16_ws_bytes(16, 11008, 4096, 0, F16) == C
    planes16 = 2 * 16 * 4096 * 2 + 2 * 2 * 43 * 128 * 256 * 4
    assert L.cbq_w8a16_ws_bytes(16, 11008, 4096, 0, F32) == C + max(planes16, 16 * 16 * 11008 * 4)
    # a weight under 8 MB keeps the general kernel at M <= 64
    assert L.cbq_w8a16_ws_bytes(16, 1024, 4096, 0, F32) == C + 16 * 16 * 1024 * 4
    assert L.cbq_w8a16_ws_bytes(4096, 11008, 4096, 0, F16) == C
    # split-K tile path, 256 CUs (also the CPU-only fallback count): 4 k-ranges
    # x 43 tiles of 128 x 256 (128 KiB of fp32 partials each)
    assert L.cbq_w8a16_ws_bytes(128, 11008, 4096, 0, F16) == C + 4 * 43 * 128 * 1024
    assert L.cbq_w8a16_ws_bytes(128, 11008, 4096, 0, _abi.BF16) == C + 4 * 43 * 128 * 1024
    # M = 256: one round of 172 tiles of 128 x 128 is modelled faster than 2
    # k-ranges x 86 tiles of 128 x 256, and needs no partials
    assert L.cbq_w8a16_ws_bytes(256, 11008, 4096, 0, F16) == C
    assert L.cbq_w8a16_ws_bytes(256, 11008, 4096, 6, _abi.BF16) == C
    assert L.cbq_w8a16_ws_bytes(512, 11008, 4096, 3, F16) == C      # 172 whole 128-row tiles
    assert L.cbq_w8a16_ws_bytes(256, 11008, 4000, 0, F16) == C      # K % 64 != 0
    # few tiles (the MLP down projection): 8 k-ranges x 32 tiles of 128 x 256,
    # 4 k-ranges x 64 tiles of 192 x 256 (192 KiB each); <= 256 workgroups
    assert L.cbq_w8a16_ws_bytes(256, 4096, 11008, 0, F16) == C + 8 * 32 * 128 * 1024
    assert L.cbq_w8a16_ws_bytes(768, 4096, 11008, 0, F16) == C + 4 * 64 * 192 * 1024
    # 24 < M <= 64 with K > 8192: the split MFMA path (11 ranges x 16 tiles of 128 x 256)
    assert L.cbq_w8a16_ws_bytes(64, 4096, 11008, 0, F16) == C + 11 * 16 * 128 * 1024
    assert L.cbq_w8a16_ws_bytes(32, 4096, 11008, 0, F16) == C + 11 * 16 * 128 * 1024
    # M = 24: k_stream<2>, no MFMA partials; fp32: the two-plane path (bf16
    # planes, then 2 planes x 8 k-ranges x 16 tiles of 128 x 256 fp32), larger
    # than the general kernel's 16 ranges of [24, 4096] fp32
    assert L.cbq_w8a16_ws_bytes(24, 4096, 11008, 0, F16) == C
    planes24 = 2 * 24 * 11008 * 2 + 2 * 8 * 16 * 128 * 256 * 4
    assert planes24 > 16 * 24 * 4096 * 4
    assert L.cbq_w8a16_ws_bytes(24, 4096, 11008, 0, F32) == C + planes24
    # K % 16 != 0 takes the general kernel whatever the dtype
    assert L.cbq_w8a16_ws_bytes(16, 11008, 4090, 0, F16) == L.cbq_w8a16_ws_bytes(
        16, 11008, 4090, 0, F32)
    # 258 tiles of 256 x 256: one full wave whole, the 2 left over split 16 ways
    assert L.cbq_w8a16_ws_bytes(1536, 11008, 4096, 0, F16) == C + 16 * 2 * 256 * 1024


def test_nd_entry_points_validate_and_size():
    """The N-D channel / group entry points: workspace sizes and argument
    checks (no device work)."""
    L = _lib()
    from cublade_amd import _abi
    C = _abi.WS_CTRL_BYTES
    # outer == 1 runs the row kernels (no workspace); inner < 512 takes the
    # column path on outer x (channels * inner), sized like axis 1; longer
    # inner runs take the segment path: [outer, channels] segment maxima plus
    # [channels] multipliers
    assert L.cbq_quant_int8_channel_nd_ws_bytes(1, 64, 128) == C
    assert L.cbq_quant_int8_channel_nd_ws_bytes(6, 40, 24) == \
        L.cbq_quant_int8_channel_ws_bytes(6, 40 * 24, 1)
    assert L.cbq_quant_int8_channel_nd_ws_bytes(6, 40, 511) == \
        L.cbq_quant_int8_channel_ws_bytes(6, 40 * 511, 1)
    assert L.cbq_quant_int8_channel_nd_ws_bytes(7, 4096, 8192) == C + 4 * (7 * 4096 + 4096)
    assert L.cbq_quant_int8_channel_nd_ws_bytes(2, 3, 512) == C + 4 * (2 * 3 + 3)
    F16 = _abi.DTYPE_CODE[torch.float16]
    dummy = ctypes.c_void_p(16)
    _einval(L.cbq_quant_int8_group_nd(dummy, F16, 2, 100, 3, 32, 1e-12, None, 0, dummy, dummy,
                                      None), "must divide")
    _einval(L.cbq_quant_int8_group_nd(dummy, F16, 2, 96, 3, 0, 1e-12, None, 0, dummy, dummy,
                                      None), "group_size")
    # group-major scale scratch: 4 bytes per scale when the tiled path can use
    # it (inner % 8 == 0, more than one group along len), else the control block
    assert L.cbq_quant_int8_group_nd_ws_bytes(1, 16384, 14336, 128) == C + 4 * 128 * 14336
    assert L.cbq_quant_int8_group_nd_ws_bytes(3, 96, 16, 32) == C + 4 * 3 * 3 * 16
    assert L.cbq_quant_int8_group_nd_ws_bytes(3, 96, 12, 32) == C     # inner % 8 != 0
    assert L.cbq_quant_int8_group_nd_ws_bytes(3, 96, 16, 96) == C     # one group along len
    assert L.cbq_quant_int8_group_nd_ws_bytes(3, 96, 1, 32) == C      # contiguous groups
    assert L.cbq_quant_int8_group_nd_ws_bytes(3, 100, 16, 32) == C    # not a divisor
    _einval(L.cbq_quant_int8_channel_nd(dummy, 9, 2, 3, 4, 1e-12, None, 0, dummy, dummy, None),
            "dtype")
    _einval(L.cbq_quant_int8_channel_nd(dummy, F16, 2, 3, 4, 1e-12, None, 0, dummy, dummy, None),
            "workspace")
    _einval(L.cbq_dequant_int8_group_nd(dummy, dummy, 2, 100, 3, 32, None, 0, dummy, F16, None),
            "must divide")
    for n in ("cbq_quant_int8_group_nd_ws_bytes", "cbq_dequant_int8_group_nd_ws_bytes"):
        f = getattr(L, n)
        assert f(2, 96, 16, 32) == C + 4 * 2 * 3 * 16 and f(2, 96, 16, 96) == C
    _einval(L.cbq_dequant_int8_channel_nd(dummy, dummy, 2, 3, 4, dummy, 0, None), "out_dtype")
    # empty shapes are no-ops
    assert L.cbq_quant_int8_group_nd(None, F16, 0, 64, 3, 32, 1e-12, None, 0, None, None,
                                     None) == 0
    assert L.cbq_dequant_int8_channel_nd(None, None, 5, 0, 3, None, F16, None) == 0


def test_mm_entry_point_validates_and_sizes():
    """cbq_mm: workspace sizes per staging case and argument checks that fail
    before any device work (the reference's wmma.cu:188-258 checks)."""
    L = _lib()
    from cublade_amd import _abi
    C = _abi.WS_CTRL_BYTES
    I8, U8, F16, BF16, F32, I32 = (_abi.I8, _abi.U8, _abi.F16, _abi.BF16, _abi.F32, _abi.I32)
    KN, NK = _abi.MM_B_KN, _abi.MM_B_NK

    def a256(v):
        return (v + 255) // 256 * 256

    # int8, B stored [N, K], K * 1 % 64 == 0: both operands read in place
    assert L.cbq_mm_ws_bytes(8192, 8192, 8192, I8, NK) == C
    # B [K, N] with K * 1 % 64 == 0: read in place by the transposing LDS reads
    assert L.cbq_mm_ws_bytes(512, 256, 128, I8, KN) == C
    assert L.cbq_mm_ws_bytes(512, 256, 128, F16, KN) == C
    # B [K, N] with K * 1 % 64 != 0: A padded, B^T staged (N rows of 128 bytes)
    assert L.cbq_mm_ws_bytes(512, 256, 80, I8, KN) == a256(a256(C + 512 * 128) + 256 * 128)
    # K * 1 % 64 != 0: both operands padded to 64-byte rows
    assert L.cbq_mm_ws_bytes(32, 48, 80, I8, NK) == a256(a256(C + 32 * 128) + 48 * 128)
    # uint8: offset copies of both plus int32 row / column sums
    assert L.cbq_mm_ws_bytes(32, 48, 64, U8, NK) == \
        a256(a256(a256(a256(C + 32 * 64) + 48 * 64) + 32 * 4) + 48 * 4)
    # fp16: 2-byte elements, K = 48 -> 96 bytes -> 128-byte rows
    assert L.cbq_mm_ws_bytes(16, 16, 48, F16, NK) == a256(a256(C + 16 * 128) + 16 * 128)
    assert L.cbq_mm_ws_bytes(16, 16, 64, BF16, NK) == C
    # few tiles: K split into 16 ranges, int32 partial planes [16, M, N]
    assert L.cbq_mm_ws_bytes(64, 1024, 4096, I8, NK) == C + 16 * 64 * 1024 * 4
    P = ctypes.c_void_p
    f = P(0x10000)
    ws = P(0x100000)
    _einval(L.cbq_mm(f, f, 9, NK, 16, 16, 16, f, I32, ws, 1 << 20, None), "unsupported dtype")
    _einval(L.cbq_mm(f, f, I8, NK, 16, 16, 16, f, F32, ws, 1 << 20, None), "int32 accumulator")
    _einval(L.cbq_mm(f, f, BF16, NK, 16, 16, 16, f, F16, ws, 1 << 20, None), "float32")
    _einval(L.cbq_mm(f, f, F16, NK, 16, 16, 16, f, I32, ws, 1 << 20, None), "float16")
    _einval(L.cbq_mm(f, f, I8, 7, 16, 16, 16, f, I32, ws, 1 << 20, None), "b_layout")
    _einval(L.cbq_mm(f, f, I8, NK, 24, 16, 16, f, I32, ws, 1 << 20, None), "multiples of 16")
    _einval(L.cbq_mm(P(0x10008), f, I8, NK, 16, 16, 16, f, I32, ws, 1 << 20, None), "aligned")
    _einval(L.cbq_mm(f, f, I8, KN, 16, 16, 16, f, I32, ws, 100, None), "workspace")
    _einval(L.cbq_mm(f, f, I8, KN, 16, 16, 16, f, I32, P(0x100010), 1 << 20, None), "workspace")
    # empty outputs are a no-op
    assert L.cbq_mm(None, None, I8, NK, 0, 16, 16, None, I32, None, 0, None) == 0


def test_loader_memoises_failures(tmp_path):
    from cublade_amd import _loader
    bad = tmp_path / "bad.hip"
    bad.write_text("this is not C++\n")
    name = "cbq_test_bad_module"
    with pytest.raises(RuntimeError, match="hipcc failed"):
        _loader.load_hip_module(name, [bad])
    assert _loader.load_error(name) is not None and not _loader.is_loaded(name)
    with pytest.raises(RuntimeError, match="failed to compile earlier"):
        _loader.load_hip_module(name, [bad])
    assert _loader.load_cuda_module is _loader.load_hip_module
    assert _loader.is_loaded("cublade_quant") or _lib() is not None


def test_quantize_tensor_host_checks():
    from cublade_amd.quantization import quantize_tensor, dequantize_tensor, QuantizedTensor
    x = torch.randn(8, 16)
    with pytest.raises(NotImplementedError):
        quantize_tensor(x, scheme="asymmetric")
    with pytest.raises(ValueError, match="No quant kernel"):
        quantize_tensor(x, dtype=torch.float8_e4m3fn, mode="group")
    with pytest.raises(ValueError, match="must be on CUDA"):
        quantize_tensor(x)
    qt = QuantizedTensor(torch.zeros(4, dtype=torch.int8), torch.ones(()), torch.zeros(()),
                         "tensor", 0, 32, torch.int8, torch.bfloat16)
    with pytest.raises(ValueError, match="must be on CUDA"):
        dequantize_tensor(qt)


def test_channel_axis_mapping():
    from cublade_amd.quantization.quantizers import channel_kernel_axis
    assert channel_kernel_axis(2, 0) == 0 and channel_kernel_axis(2, 1) == 1
    assert channel_kernel_axis(2, -1) == 1 and channel_kernel_axis(3, -1) == 1
    assert channel_kernel_axis(1, 0) == 0 and channel_kernel_axis(1, -1) == 0
    assert channel_kernel_axis(3, 1) == 2 and channel_kernel_axis(4, -2) == 2   # N-D path
    with pytest.raises(IndexError):
        channel_kernel_axis(3, 3)
    with pytest.raises(IndexError):
        channel_kernel_axis(3, -4)


def test_outlier_utils_match_definition():
    from cublade_amd.quantization import (detect_outlier_columns, separate_outliers,
                                          split_weights_by_outliers)
    w = torch.zeros(4, 10)
    w[1, 3] = 6.5
    w[2, 7] = -7.0
    w[0, 5] = 6.0            # not > threshold
    w[3, 9] = float("nan")   # NaN never counts
    assert detect_outlier_columns(w, 6.0) == [3, 7]
    wn, wo, nc, oc = split_weights_by_outliers(w, [7, 3])
    assert nc == [0, 1, 2, 4, 5, 6, 8, 9] and oc == [7, 3]
    assert torch.equal(wo, w[:, [7, 3]], ) and wn.shape == (4, 8)
    wn, wo, nc, oc = separate_outliers(w, 6.0)
    assert oc == [3, 7] and wo.shape == (4, 2)


def test_replace_linear_layers_filters():
    from cublade_amd.quantization import replace_linear_layers

    class Fake(nn.Module):
        def __init__(self, in_f, out_f, bias=True, dtype=torch.float32, **kw):
            super().__init__()
            self.shape, self.kw, self.dtype_ = (in_f, out_f), kw, dtype
            self.bias = None
            self.got = None

        def quantize(self, w):
            self.got = w

    model = nn.Sequential()
    model.add_module("q_proj", nn.Linear(4, 8))
    model.add_module("k_proj", nn.Linear(4, 8, bias=False))
    inner = nn.Sequential()
    inner.add_module("lm_head", nn.Linear(8, 3))
    inner.add_module("v_proj", nn.Linear(8, 3).half())
    model.add_module("inner", inner)
    replace_linear_layers(model, Fake, target_modules=["proj"], exclude_modules=["k_"],
                          quant_kwargs={"handle_outliers": True})
    assert isinstance(model.q_proj, Fake) and model.q_proj.kw == {"handle_outliers": True}
    assert isinstance(model.k_proj, nn.Linear)
    assert isinstance(model.inner.lm_head, nn.Linear)
    assert isinstance(model.inner.v_proj, Fake) and model.inner.v_proj.dtype_ == torch.float16
    assert model.q_proj.got is not None and model.q_proj.bias is not None


def _cpu_layer(K, N, dt, bias, seed, outliers=()):
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    g = torch.Generator().manual_seed(seed)
    layer = cuBladeW8A16LinearLayer(K, N, bias=bias, dtype=dt, handle_outliers=bool(outliers))
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    oc = list(outliers)
    if oc:
        wq[:, oc] = 0
        layer.outlier_cols = torch.tensor(oc, dtype=torch.long)
        layer.normal_cols = torch.tensor([c for c in range(K) if c not in oc], dtype=torch.long)
        layer.outlier_weights = (0.5 * torch.randn(N, len(oc), generator=g)).to(dt)
    layer.int8_weights = wq
    layer.scales = (torch.rand(N, generator=g) * 0.01).to(dt)
    if bias:
        layer.bias.data = (0.1 * torch.randn(N, generator=g)).to(dt)
    return layer


@pytest.mark.parametrize("outliers", [(), (1, 9, 30)])
def test_layer_cpu_branch_matches_oracle(outliers):
    layer = _cpu_layer(40, 24, torch.float32, True, 3, outliers)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 40, generator=g)
    y = layer(x)
    assert y.shape == (2, 3, 24)
    ref = oracle.w8a16_linear(x.reshape(-1, 40).numpy(), oracle.F32, layer.int8_weights.numpy(),
                              layer.scales.numpy(), bias=layer.bias.detach().numpy(),
                              outlier_cols=np.array(outliers, np.int64) if outliers else None,
                              w_out=layer.outlier_weights.numpy() if outliers else None)
    np.testing.assert_allclose(y.reshape(-1, 24).detach().numpy(), ref, rtol=1e-5, atol=1e-5)


def test_state_dict_compact_layout_expands():
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    src = _cpu_layer(16, 6, torch.float16, True, 7, outliers=(2, 11))
    sd = src.state_dict()                 # the reference layout [out, in - n_out]
    assert tuple(sd["int8_weights"].shape) == (6, 14)
    dst = cuBladeW8A16LinearLayer(16, 6, bias=True, dtype=torch.float16, handle_outliers=True)
    dst.load_state_dict(sd)
    assert torch.equal(dst.int8_weights, src.int8_weights)
    assert torch.equal(dst.outlier_cols, src.outlier_cols)
    x = torch.randn(3, 16)
    torch.testing.assert_close(dst(x), src(x))


def test_state_dict_saves_reference_layout():
    """With outliers, state_dict() holds the reference's compact
    int8_weights [out, in - n_out] (linear.py:48-66); without, [out, in]."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    src = _cpu_layer(16, 6, torch.float16, True, 7, outliers=(2, 11))
    sd = src.state_dict()
    assert tuple(sd["int8_weights"].shape) == (6, 14)
    assert torch.equal(sd["int8_weights"], src.int8_weights[:, src.normal_cols])
    assert tuple(src.int8_weights.shape) == (6, 16)          # memory layout unchanged
    assert set(sd) == {"int8_weights", "scales", "outlier_weights", "normal_cols",
                       "outlier_cols", "bias"}
    dst = cuBladeW8A16LinearLayer(16, 6, bias=True, dtype=torch.float16, handle_outliers=True)
    dst.load_state_dict(sd)
    assert torch.equal(dst.int8_weights, src.int8_weights)
    plain = _cpu_layer(16, 6, torch.float16, True, 8, outliers=())
    assert tuple(plain.state_dict()["int8_weights"].shape) == (6, 16)


def test_oracle_not_imported_by_product():
    """The product packages never import the oracle (test infrastructure)."""
    for pkg in ("cublade_amd", "cublade"):
        for p in (ROOT / pkg).rglob("*.py"):
            text = p.read_text()
            assert "import oracle" not in text and "from oracle" not in text, p


def test_reference_import_name_resolves_without_gpu():
    """``cublade.*`` (the reference's import name, quantization/__init__.py:1-17,
    bindings/cuda/__init__.py:1-4, _loader.py:24-125) names the modules of
    cublade_amd themselves, with bindings.cuda -> bindings.hip."""
    import importlib

    import cublade
    import cublade_amd
    from cublade.quantization import (QuantizedTensor, cuBladeW8A16LinearLayer,
                                      dequantize_tensor, detect_outlier_columns, quantize_model,
                                      quantize_tensor, separate_outliers,
                                      split_weights_by_outliers)
    from cublade._loader import CSRC, is_loaded, load_cuda_module, load_error
    from cublade.bindings.cuda.quantize_fp8 import quantize_per_tensor_fp8
    from cublade.bindings.cuda.dequantize_int8 import dequantize_per_group_int8
    q = cublade_amd.quantization
    assert (quantize_tensor, dequantize_tensor, QuantizedTensor, quantize_model) == (
        q.quantize_tensor, q.dequantize_tensor, q.QuantizedTensor, q.quantize_model)
    assert cuBladeW8A16LinearLayer is q.cuBladeW8A16LinearLayer
    assert (detect_outlier_columns, separate_outliers, split_weights_by_outliers) == (
        q.detect_outlier_columns, q.separate_outliers, q.split_weights_by_outliers)
    assert load_cuda_module is cublade_amd._loader.load_hip_module
    assert CSRC == cublade_amd._loader.CSRC and is_loaded is cublade_amd._loader.is_loaded
    assert load_error is cublade_amd._loader.load_error
    assert quantize_per_tensor_fp8 is cublade_amd.bindings.hip.quantize_per_tensor_fp8
    assert dequantize_per_group_int8 is cublade_amd.bindings.hip.dequantize_per_group_int8
    assert cublade.bindings.cuda is cublade_amd.bindings.hip
    assert importlib.import_module("cublade.quantization.linear") is \
        importlib.import_module("cublade_amd.quantization.linear")
    # the real module keeps its own spec
    assert cublade.quantization.__spec__.name == "cublade_amd.quantization"
    assert cublade.quantize_tensor is quantize_tensor
    assert cublade.quantize_per_tensor_int8 is cublade_amd.bindings.hip.quantize_per_tensor_int8
    for missing in ("cublade.kernels", "cublade.bindings.triton"):
        with pytest.raises(ImportError):
            importlib.import_module(missing)


def test_activation_outlier_columns_and_mode_checks():
    """LLM.int8's activation criterion (opt-in layer mode): a feature is an
    outlier when any |x| in it is > threshold (strict), NaN never counts,
    every leading dimension is reduced; the layer rejects an unknown mode
    and an activation mode without a calibration batch before any GPU work."""
    from cublade_amd.quantization import (cuBladeW8A16LinearLayer,
                                          detect_activation_outlier_columns)
    x = torch.zeros(2, 3, 8)
    x[0, 1, 2] = 6.5
    x[1, 2, 5] = -7.0
    x[0, 0, 4] = 6.0                 # not > threshold
    x[1, 0, 7] = float("nan")
    assert detect_activation_outlier_columns(x, 6.0) == [2, 5]
    assert detect_activation_outlier_columns(x, 7.5) == []
    with pytest.raises(ValueError, match="outlier_mode"):
        cuBladeW8A16LinearLayer(8, 4, outlier_mode="rows")
    layer = cuBladeW8A16LinearLayer(8, 4, handle_outliers=True, outlier_mode="activation")
    with pytest.raises(ValueError, match="calibration batch"):
        layer.quantize(torch.zeros(4, 8))
    with pytest.raises(ValueError, match="calibration batch"):
        layer.quantize(torch.zeros(4, 8), activations=torch.zeros(3, 7))


def test_benchmark_returns_the_reference_contract(capsys):
    """cublade.benchmark.benchmark keeps the reference's signature (n_flop a
    required keyword) and result dict (benchmark/core.py:5-71): keys
    kernel.{time_ms, gflops, max_err, passed, output} and
    reference.{time_ms, gflops, output}, plus the printed table."""
    import inspect

    from cublade_amd.benchmark import benchmark

    sig = inspect.signature(benchmark)
    assert sig.parameters["n_flop"].kind is inspect.Parameter.KEYWORD_ONLY
    assert sig.parameters["n_flop"].default is inspect.Parameter.empty
    for name, default in (("warmup", 1), ("atol", 1e-5), ("rtol", 1e-3)):
        assert sig.parameters[name].default == default
    a = torch.randn(64, 64)

    def ref(x):
        return x @ x

    def kern(x):
        return torch.mm(x, x)

    with pytest.raises(TypeError):
        benchmark(kern, ref, a)
    res = benchmark(kern, ref, a, n_flop=2 * 64 ** 3, reps=3)
    assert set(res) == {"kernel", "reference"}
    assert set(res["kernel"]) == {"time_ms", "gflops", "max_err", "passed", "output"}
    assert set(res["reference"]) == {"time_ms", "gflops", "output"}
    assert res["kernel"]["passed"] is True and res["kernel"]["max_err"] < 1e-3
    assert res["kernel"]["time_ms"] > 0 and res["reference"]["gflops"] > 0
    out = capsys.readouterr().out
    assert "GFLOPS" in out and "PASS" in out and "REF" in out
