"""Seeded random sweep of the public API on the GPU against the CPU oracle.

Each case draws a rank (1-4), a shape, an input dtype, a mode, an axis, a
group size that divides the axis and, for some cases, a view whose data
pointer is off the 16-byte grid (a contiguous slice of a larger buffer).
Bar as in test_gpu_quant: bit-exact codes, scales and dequantized outputs
(any NaN matches any NaN). The W8A16 part draws M, K, N, the activation
dtype, bias and outlier columns and checks rtol = atol = 1e-2 against the
oracle's exact accumulation; its streaming part draws the weight-streaming
range (M <= 64, K a multiple of 1024, 8-64 MB of int8 weight), checks
sampled rows against the oracle and every row against a float32 product on
the GPU; its tile part draws M in (64, 384) with K a multiple of 64 and a
ragged N (the 128 x 128 tiles or a split plan, and the same call without a
workspace). The cases are fixed by their seeds, so a failure names a
reproducible case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests._util import (CODE_OF, DTYPE_OF, assert_array_equal, assert_bits_equal_16,
                         assert_fp8_equal, bits, from_bits)

pytestmark = pytest.mark.gpu

DEV = "cuda"
N_QUANT_CASES = 160
N_W8A16_CASES = 64


def _shape(rng, max_numel=1 << 17):
    nd = int(rng.integers(1, 5))
    while True:
        shape = tuple(int(rng.choice([1, 2, 3, 5, 8, 16, 24, 32, 64, 96, 128, 257, 520, 1024]))
                      for _ in range(nd))
        if 0 < int(np.prod(shape)) <= max_numel:
            return shape


def _upload(x_bits, code, shape, offset):
    """x on the device as a contiguous tensor; offset > 0 makes it a slice
    that starts `offset` elements into a larger buffer."""
    t = from_bits(x_bits.reshape(-1), code, "cpu")
    if offset:
        buf = torch.zeros(t.numel() + offset, dtype=t.dtype)
        buf[offset:] = t
        return buf.to(DEV)[offset:].view(shape)
    return t.to(DEV).view(shape)


def _quant_case(i):
    rng = np.random.default_rng(1000 + i)
    mode = ["tensor", "tensor_fp8", "channel", "group"][i % 4]
    shape = _shape(rng)
    code = int(rng.choice([oracle.BF16, oracle.F16] if mode == "tensor_fp8"
                          else [oracle.BF16, oracle.F16, oracle.F32]))
    nd = len(shape)
    axis = int(rng.integers(-nd, nd))
    F = shape[axis]
    divs = [g for g in range(1, F + 1) if F % g == 0]
    G = int(rng.choice(divs))
    offset = int(rng.choice([0, 0, 1, 3]))
    scale = float(rng.choice([1e-3, 1.0, 40.0]))
    return mode, shape, code, axis, G, offset, scale


def _out_code(code):
    return oracle.BF16 if code == oracle.F32 else code


@pytest.mark.parametrize("i", range(N_QUANT_CASES))
def test_random_quant_dequant(i):
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    mode, shape, code, axis, G, offset, scale = _quant_case(i)
    print(f"[random quant {i}] mode={mode} shape={shape} code={code} axis={axis} G={G} "
          f"offset={offset}", flush=True)
    g = torch.Generator().manual_seed(i)
    v = torch.randn(*shape, generator=g) * scale
    if v.numel() > 4:
        v.view(-1)[int(torch.randint(0, v.numel(), (1,), generator=g))] *= 50.0
    x = bits(v.to(DTYPE_OF[code]))
    xt = _upload(x, code, shape, offset)
    out = _out_code(code)

    if mode == "tensor_fp8":
        qt = quantize_tensor(xt, dtype=torch.float8_e4m3fn, mode="tensor")
        qo, so = oracle.quant_fp8_tensor(x.reshape(-1), code)
        assert_fp8_equal(bits(qt.data), qo, "fp8 q")
        assert_array_equal(bits(qt.scale).reshape(-1).view(np.uint32),
                           np.array([so], np.float32).view(np.uint32), "fp8 scale")
        yo = oracle.dequant_fp8_tensor(qo, so, out)
    elif mode == "tensor":
        qt = quantize_tensor(xt, dtype=torch.int8, mode="tensor")
        qo, so = oracle.quant_int8_tensor(x.reshape(-1), code)
        assert_array_equal(bits(qt.data), qo, "int8 q")
        assert_array_equal(bits(qt.scale).reshape(-1).view(np.uint32),
                           np.array([so], np.float32).view(np.uint32), "int8 scale")
        yo = oracle.dequant_int8_tensor(qo, so, out)
    elif mode == "channel":
        qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=axis)
        C = shape[axis]
        ax = axis % len(shape)
        mshape = (C,) + tuple(d for j, d in enumerate(shape) if j != ax)
        moved = np.ascontiguousarray(np.moveaxis(x, ax, 0)).reshape(C, -1)
        qo, so = oracle.quant_int8_channel(moved, code, axis=0)
        assert_array_equal(bits(qt.data), np.moveaxis(qo.reshape(mshape), 0, ax), "channel q")
        assert_array_equal(bits(qt.scale).view(np.uint32),
                           np.asarray(so, np.float32).view(np.uint32), "channel scale")
        yo = np.moveaxis(oracle.dequant_int8_channel(qo, so, out, axis=0).reshape(mshape), 0, ax)
    else:
        qt = quantize_tensor(xt, dtype=torch.int8, mode="group", group_size=G, ch_axis=axis)
        ax = axis % len(shape)
        moved = np.ascontiguousarray(np.moveaxis(x, ax, -1))
        qo, so = oracle.quant_int8_group(moved.reshape(-1, G), code, G)
        assert_array_equal(bits(qt.data), np.moveaxis(qo.reshape(moved.shape), -1, ax), "group q")
        assert_array_equal(bits(qt.scale).view(np.uint32),
                           np.asarray(so, np.float32).view(np.uint32), "group scale")
        yo = np.moveaxis(oracle.dequant_int8_group(qo, so, G, out).reshape(moved.shape), -1, ax)

    qt.original_dtype = DTYPE_OF[out]
    y = dequantize_tensor(qt)
    assert y.dtype == DTYPE_OF[out] and tuple(y.shape) == shape
    assert_bits_equal_16(bits(y), yo, out, f"{mode} y")


def _w8a16_case(i):
    rng = np.random.default_rng(5000 + i)
    M = int(rng.choice([1, 2, 7, 16, 17, 33, 64, 65, 130, 256, 300, 513]))
    K = int(rng.choice([16, 48, 64, 100, 128, 250, 512, 1024, 1040]))
    N = int(rng.choice([1, 17, 48, 64, 100, 256, 300, 520]))
    dt = [torch.float16, torch.bfloat16][i % 2]
    bias = bool(rng.integers(0, 2))
    n_out = int(rng.choice([0, 0, 1, 3])) if K >= 8 else 0
    return M, K, N, dt, bias, n_out


@pytest.mark.parametrize("i", range(N_W8A16_CASES))
def test_random_w8a16(i):
    from cublade_amd.bindings.hip import w8a16_linear
    M, K, N, dt, bias, n_out = _w8a16_case(i)
    print(f"[random w8a16 {i}] M={M} K={K} N={N} dt={dt} bias={bias} n_out={n_out}", flush=True)
    g = torch.Generator().manual_seed(7000 + i)
    x = torch.randn(M, K, generator=g)
    oc = sorted(torch.randperm(K, generator=g)[:n_out].tolist()) if n_out else []
    w = 0.02 * torch.randn(N, K, generator=g)
    if oc:
        x[:, oc] = 10.0 * torch.sign(torch.randn(M, len(oc), generator=g))
    wn = w.clone()
    if oc:
        wn[:, oc] = 0
    inv = torch.tensor(127.0) / torch.clamp(wn.abs().amax(dim=1), min=1e-12)
    wq = torch.round(wn * inv[:, None]).clamp(-127, 127).to(torch.int8)
    s = (1.0 / inv).to(dt)
    b = (0.1 * torch.randn(N, generator=g)).to(dt) if bias else None
    w_out = w[:, oc].to(dt) if oc else None
    xd = x.to(dt)
    y = w8a16_linear(xd.to(DEV), wq.to(DEV), s.to(DEV), None if b is None else b.to(DEV),
                     torch.tensor(oc, dtype=torch.int64, device=DEV) if oc else None,
                     None if w_out is None else w_out.to(DEV))
    assert y.dtype == dt and tuple(y.shape) == (M, N)
    ref = oracle.w8a16_linear(bits(xd), CODE_OF[dt], wq.numpy(), bits(s),
                              bias=None if b is None else bits(b),
                              outlier_cols=np.asarray(oc, np.int64) if oc else None,
                              w_out=None if w_out is None else bits(w_out))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-2)


N_STREAM_CASES = 16


def _stream_case(i):
    """Shapes of the weight-streaming range: M <= 64, K a multiple of 1024
    and a weight of 8-64 MB (k_stream1 / k_stream; K > 4096 also reaches
    k_skinny and, for M > 24 with K > 8192, the split MFMA tile path)."""
    rng = np.random.default_rng(9000 + i)
    Ms = [1, 2, 3, 5, 8, 13, 16, 17, 24, 25, 31, 32, 33, 48, 49, 63, 64]
    M = Ms[(3 * i) % len(Ms)]
    K = [1024, 2048, 3072, 4096, 5120, 8192, 12288][i % 7]
    n_min = -(-(8 << 20) // K)
    N = int(rng.integers(n_min, max(n_min + 1, (64 << 20) // K)))
    N -= N % int(rng.choice([1, 1, 16, 256]))
    N = max(N, n_min)
    dt = [torch.float16, torch.bfloat16][i % 2]
    bias = bool(rng.integers(0, 2))
    n_out = int(rng.choice([0, 0, 1, 2, 5]))
    return M, K, N, dt, bias, n_out


@pytest.mark.parametrize("i", range(N_STREAM_CASES))
def test_random_w8a16_streaming(i):
    """int8 codes drawn directly (uniform over [-127, 127]) with scales that
    keep |y| near 1; four sampled rows against the oracle's exact
    accumulation and every row against a float32 product of the dequantized
    weight on the GPU, both at rtol = atol = 1e-2."""
    from cublade_amd.bindings.hip import w8a16_linear
    M, K, N, dt, bias, n_out = _stream_case(i)
    print(f"[random w8a16 streaming {i}] M={M} K={K} N={N} dt={dt} bias={bias} "
          f"n_out={n_out}", flush=True)
    g = torch.Generator().manual_seed(11000 + i)
    x = torch.randn(M, K, generator=g)
    oc = sorted(torch.randperm(K, generator=g)[:n_out].tolist()) if n_out else []
    if oc:
        x[:, oc] = 10.0 * torch.sign(torch.randn(M, len(oc), generator=g))
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    if oc:
        wq[:, oc] = 0
    s = ((0.5 + torch.rand(N, generator=g)) / (73.0 * K ** 0.5)).to(dt)
    b = (0.1 * torch.randn(N, generator=g)).to(dt) if bias else None
    w_out = (0.02 * torch.randn(N, len(oc), generator=g)).to(dt) if oc else None
    xd = x.to(dt)
    xg, wg, sg = xd.to(DEV), wq.to(DEV), s.to(DEV)
    bg = None if b is None else b.to(DEV)
    og = torch.tensor(oc, dtype=torch.int64, device=DEV) if oc else None
    wog = None if w_out is None else w_out.to(DEV)
    y = w8a16_linear(xg, wg, sg, bg, og, wog)
    assert y.dtype == dt and tuple(y.shape) == (M, N)

    rows = np.unique(np.array([0, M - 1, M // 2, (7 * i) % M], np.int64))
    ref = oracle.w8a16_linear(bits(xd), CODE_OF[dt], wq.numpy(), bits(s),
                              bias=None if b is None else bits(b),
                              outlier_cols=np.asarray(oc, np.int64) if oc else None,
                              w_out=None if w_out is None else bits(w_out), rows=rows)
    np.testing.assert_allclose(y.float().cpu().numpy()[rows], ref, rtol=1e-2, atol=1e-2)

    wf = wg.float() * sg.float()[:, None]
    ref_all = xg.float() @ wf.t()
    if oc:
        ref_all += xg.float()[:, og] @ wog.float().t()
    if bg is not None:
        ref_all += bg.float()
    torch.testing.assert_close(y.float(), ref_all, rtol=1e-2, atol=1e-2)


N_TILE_CASES = 16


def _tile_case(i):
    """Shapes of the MFMA tile path below 384 rows (128 x 128 tiles, or a
    split plan where the host's model prefers one): M in (64, 384), K a
    multiple of 64, N ragged."""
    rng = np.random.default_rng(13000 + i)
    M = int(rng.integers(65, 384))
    K = 64 * int(rng.integers(1, 97))
    N = int(rng.integers(16, 6000))
    dt = [torch.float16, torch.bfloat16][i % 2]
    bias = bool(rng.integers(0, 2))
    n_out = int(rng.choice([0, 0, 1, 6, 17])) if K >= 32 else 0
    return M, K, N, dt, bias, n_out


@pytest.mark.parametrize("i", range(N_TILE_CASES))
def test_random_w8a16_tiles(i):
    """Four sampled rows against the oracle's exact accumulation and every
    row against a float32 product of the dequantized weight on the GPU, at
    rtol = atol = 1e-2, with and without a workspace (the split plans need
    one; the 128 x 128 tiles do not)."""
    from cublade_amd import _abi
    from cublade_amd.bindings.hip import w8a16_linear
    M, K, N, dt, bias, n_out = _tile_case(i)
    print(f"[random w8a16 tiles {i}] M={M} K={K} N={N} dt={dt} bias={bias} n_out={n_out}",
          flush=True)
    g = torch.Generator().manual_seed(15000 + i)
    x = torch.randn(M, K, generator=g)
    oc = sorted(torch.randperm(K, generator=g)[:n_out].tolist()) if n_out else []
    if oc:
        x[:, oc] = 10.0 * torch.sign(torch.randn(M, len(oc), generator=g))
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    if oc:
        wq[:, oc] = 0
    s = ((0.5 + torch.rand(N, generator=g)) / (73.0 * K ** 0.5)).to(dt)
    b = (0.1 * torch.randn(N, generator=g)).to(dt) if bias else None
    w_out = (0.02 * torch.randn(N, len(oc), generator=g)).to(dt) if oc else None
    xd = x.to(dt)
    xg, wg, sg = xd.to(DEV), wq.to(DEV), s.to(DEV)
    bg = None if b is None else b.to(DEV)
    og = torch.tensor(oc, dtype=torch.int64, device=DEV) if oc else None
    wog = None if w_out is None else w_out.to(DEV)
    y = w8a16_linear(xg, wg, sg, bg, og, wog)
    assert y.dtype == dt and tuple(y.shape) == (M, N)

    rows = np.unique(np.array([0, M - 1, M // 2, (11 * i) % M], np.int64))
    ref = oracle.w8a16_linear(bits(xd), CODE_OF[dt], wq.numpy(), bits(s),
                              bias=None if b is None else bits(b),
                              outlier_cols=np.asarray(oc, np.int64) if oc else None,
                              w_out=None if w_out is None else bits(w_out), rows=rows)
    np.testing.assert_allclose(y.float().cpu().numpy()[rows], ref, rtol=1e-2, atol=1e-2)

    wf = wg.float() * sg.float()[:, None]
    ref_all = xg.float() @ wf.t()
    if oc:
        ref_all += xg.float()[:, og] @ wog.float().t()
    if bg is not None:
        ref_all += bg.float()
    torch.testing.assert_close(y.float(), ref_all, rtol=1e-2, atol=1e-2)

    # the same call with only the control block as workspace (no split)
    L = _abi.lib()
    y_one = torch.empty_like(y)
    ws = torch.zeros(_abi.WS_CTRL_BYTES, dtype=torch.uint8, device=DEV)
    rc = L.cbq_w8a16_linear(_abi.ptr(xg), CODE_OF[dt], _abi.ptr(wg), _abi.ptr(sg),
                            None if bg is None else _abi.ptr(bg),
                            None if og is None else _abi.ptr(og), n_out,
                            None if wog is None else _abi.ptr(wog), M, N, K, _abi.ptr(ws),
                            ws.numel(), _abi.ptr(y_one), _abi.stream_handle(xg.device))
    assert rc == 0
    torch.testing.assert_close(y_one.float(), ref_all, rtol=1e-2, atol=1e-2)
