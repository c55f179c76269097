"""GPU parity of the W8A16 linear (HIP C ABI via the binding and the layer)
against the oracle's exact-accumulation W8A16 (float64) and the golden
vectors. Gate (north star): rtol 1e-2 / atol 1e-2.

Covers the MFMA path (fp16 / bf16, M / N / K tails), fp32 activations on the
matrix cores as two bf16 planes (M > 64, K % 64 == 0), the general path (other
fp32 shapes, K not a multiple of 16, unaligned activations), bias, the
outlier side-GEMM, quantize_model on an MLP, state_dict round trips (own and
reference compact layout) and the BASELINE config-5 shapes (row subsets
against the oracle, full output against a GPU fp32 matmul of the same
operands).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from tests import _golden as G
from tests._util import CODE_OF, DTYPE_OF, bits, from_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(rtol=1e-2, atol=1e-2)


@pytest.fixture(scope="module", autouse=True)
def _loaded():
    from cublade_amd import _abi
    _abi.lib()


def w8a16(*args, **kw):
    from cublade_amd.bindings.hip import w8a16_linear
    return w8a16_linear(*args, **kw)


def expand_compact(wq_c: np.ndarray, normal_cols, K: int) -> np.ndarray:
    full = np.zeros((wq_c.shape[0], K), np.int8)
    full[:, normal_cols] = wq_c
    return full


def oracle_y(x, code, wq_full, scales, bias=None, oc=None, w_out=None, rows=None):
    """Oracle on the full-K weight (outlier columns are zero in wq_full)."""
    return oracle.w8a16_linear(x, code, wq_full, scales, bias=bias,
                               outlier_cols=None if oc is None else np.asarray(oc, np.int64),
                               w_out=w_out, rows=rows)


def make_case(M, K, N, dt, seed, bias=False, n_out=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    oc = sorted(torch.randperm(K, generator=g)[:n_out].tolist()) if n_out else []
    w = 0.02 * torch.randn(N, K, generator=g)
    if oc:
        x[:, oc] = 10.0 * torch.sign(torch.randn(M, len(oc), generator=g))
        w[:, oc] *= 400.0
    wn = w.clone()
    if oc:
        wn[:, oc] = 0
    amax = wn.abs().amax(dim=1)
    inv = torch.tensor(127.0) / torch.clamp(amax, min=1e-12)
    wq = torch.round(wn * inv[:, None]).clamp(-127, 127).to(torch.int8)
    s = (1.0 / inv).to(dt)
    b = (0.1 * torch.randn(N, generator=g)).to(dt) if bias else None
    w_out = w[:, oc].to(dt) if oc else None
    return x.to(dt), wq, s, b, oc, w_out


def run_and_check(M, K, N, dt, seed, bias=False, n_out=0, rows=None, x_offset=0):
    x, wq, s, b, oc, w_out = make_case(M, K, N, dt, seed, bias, n_out)
    code = CODE_OF[dt]
    if x_offset:
        xbuf = torch.zeros(M * K + x_offset, dtype=dt, device=DEV)
        xbuf[x_offset:] = x.reshape(-1).to(DEV)
        xd = xbuf[x_offset:].view(M, K)
    else:
        xd = x.to(DEV)
    y = w8a16(xd, wq.to(DEV), s.to(DEV), None if b is None else b.to(DEV),
              torch.tensor(oc, dtype=torch.int64, device=DEV) if oc else None,
              None if w_out is None else w_out.to(DEV))
    assert y.dtype == dt and tuple(y.shape) == (M, N)
    r = None if rows is None else np.asarray(rows, np.int64)
    ref = oracle_y(bits(x), code, wq.numpy(), bits(s), None if b is None else bits(b),
                   oc or None, None if w_out is None else bits(w_out), rows=r)
    got = y.float().cpu().numpy()
    if r is not None:
        got = got[r]
    np.testing.assert_allclose(got, ref, **TOL)
    return y


@pytest.mark.parametrize("meta,arr", G.cases("w8a16"), ids=G.ids("w8a16"))
def test_golden(meta, arr):
    M, K, N = meta["shape"]
    dt = DTYPE_OF[meta["dtype"]]
    wq = arr["wq"]
    oc = arr.get("outlier_cols")
    if oc is not None:
        wq = expand_compact(wq, arr["normal_cols"], K)
    y = w8a16(from_bits(arr["x"].reshape(-1), meta["dtype"], DEV).view(M, K),
              torch.from_numpy(wq).to(DEV),
              from_bits(arr["scales"], meta["dtype"], DEV),
              None if "bias" not in arr else from_bits(arr["bias"], meta["dtype"], DEV),
              None if oc is None else torch.from_numpy(oc).to(DEV),
              None if oc is None else from_bits(arr["w_out"].reshape(-1), meta["dtype"],
                                                DEV).view(N, len(oc)))
    np.testing.assert_allclose(y.float().cpu().numpy(), arr["y"], **TOL)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", [(1, 64, 48), (16, 128, 128), (7, 4096, 96),     # skinny, TM 1
                                   (24, 128, 96), (40, 256, 200), (64, 64, 64),    # skinny, TM 2 / 4
                                   (100, 96, 200), (128, 256, 128), (129, 80, 130),
                                   (256, 512, 384), (300, 160, 257),               # 128 x 64 tiles
                                   (1030, 128, 300), (1024, 320, 512),             # DMA 256 x 256
                                   (1031, 192, 1000), (1024, 64, 256), (1290, 448, 520),
                                   (1024, 80, 300), (1100, 208, 264),              # K % 64 != 0
                                   (7, 2048, 8200), (1, 4096, 4000), (13, 1024, 9000),  # k_stream1
                                   (16, 1024, 14336), (5, 2048, 16384), (16, 4096, 12301),  # 64 rows
                                   (24, 4096, 5000), (64, 2048, 6000), (40, 1024, 9000),  # k_stream
                                   (200, 4096, 1000), (700, 1024, 3000), (500, 2048, 2600),  # split-K
                                   (800, 256, 3000)])                               # DMA, M < 1024
def test_mfma_shapes(dt, M, K, N):
    run_and_check(M, K, N, dt, seed=M * 31 + K + N, bias=(M % 2 == 1))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_outlier_side_gemm(dt):
    run_and_check(64, 256, 96, dt, seed=5, bias=True, n_out=6)
    run_and_check(130, 512, 200, dt, seed=6, bias=False, n_out=17)
    run_and_check(1100, 256, 300, dt, seed=7, bias=True, n_out=5)      # DMA tile kernel
    run_and_check(16, 2048, 4400, dt, seed=8, bias=True, n_out=4)      # k_stream1
    run_and_check(40, 1024, 9000, dt, seed=9, bias=False, n_out=3)     # k_stream


@pytest.mark.parametrize("M,K,N", [(5, 100, 40), (33, 24, 17)])
def test_general_path_odd_k(M, K, N):
    run_and_check(M, K, N, torch.float16, seed=K, bias=True)
    run_and_check(M, K, N, torch.bfloat16, seed=K + 1, n_out=3)


def test_general_path_fp32_and_unaligned():
    run_and_check(20, 128, 64, torch.float32, seed=2, bias=True, n_out=2)
    run_and_check(40, 256, 72, torch.float16, seed=3, bias=True, x_offset=3)


@pytest.mark.parametrize("M,K,N", [(16, 4096, 1024), (300, 1000, 700), (65, 4097, 130),
                                   (1, 33, 1)])
def test_general_path_fp32_tiles(M, K, N):
    """fp32 activations at both tile heights (16 and 64 rows), partial tiles
    in every dimension and K tails that are not a multiple of the 32-k step."""
    run_and_check(M, K, N, torch.float32, seed=M + K, bias=True, n_out=3 if K > 3 else 0,
                  rows=list(range(0, M, max(1, M // 7))))
    run_and_check(M, K, N, torch.bfloat16, seed=M + K + 1, x_offset=1 if K % 2 else 0)


@pytest.mark.parametrize("M,K,N", [(65, 64, 40), (300, 1024, 700), (1100, 256, 520),
                                   (2137, 2048, 8192), (16, 4096, 2048), (1, 8192, 1024),
                                   (40, 2048, 4160), (64, 11008, 1024), (5160, 4096, 11008)])
def test_fp32_two_plane_path(M, K, N):
    """fp32 activations with K % 64 == 0, no outlier columns and M > 64 (or
    M <= 64 with a weight of at least 8 MB, then K also split into up to 8
    ranges per plane) run on the matrix cores as two bf16 planes of x (hi
    truncated, lo = bf16(x - hi)) against the int8 weights; M = 5160 at
    N = 11008 exceeds the path's 256 MiB workspace cap and runs as chunks of
    2560 and 2600 rows (the 40-row remainder joins the last chunk). Sampled rows
    against the oracle; the whole output against a float64 product within
    2^-14 of sum_k |x w s| (x keeps 16 significant bits; dropping the lo plane
    would leave only 8); with outlier columns the VALU kernel runs, also
    against the oracle."""
    from cublade_amd import _abi
    assert _abi.lib().cbq_w8a16_ws_bytes(M, N, K, 0, _abi.DTYPE_CODE[torch.float32]) > \
        _abi.WS_CTRL_BYTES + 2 * M * K * 2
    print(f"[w8a16 fp32 planes] M={M} K={K} N={N}", flush=True)
    rows = [0, M // 3, M - 1]
    y = run_and_check(M, K, N, torch.float32, seed=M + 7, bias=True, rows=rows)
    x, wq, s, b, _, _ = make_case(M, K, N, torch.float32, M + 7, True, 0)
    xd, wd, sd, bd = (t.to(DEV) for t in (x, wq, s, b))
    prod = xd.double() @ wd.double().t().contiguous()
    ref = prod * sd.double() + bd.double()
    bound = (xd.double().abs() @ wd.double().abs().t().contiguous()) * sd.double() * 2.0 ** -14
    err = (y.double() - ref).abs()
    assert bool((err <= bound + 1e-6).all()), float((err - bound).max())
    run_and_check(M, K, N, torch.float32, seed=M + 8, n_out=2, rows=rows)


def test_fp32_two_plane_path_special_values():
    """NaN, +-inf and huge finite activations: the two-plane path and the VALU
    kernel (forced by a control-block-only workspace) give the same NaN and
    inf pattern and close finite values."""
    from cublade_amd import _abi
    M, K, N = 130, 256, 96
    x, wq, s, _, _, _ = make_case(M, K, N, torch.float32, 31, False, 0)
    x[3, 5] = float("nan")
    x[7, 9] = float("inf")
    x[8, 1] = -float("inf")
    x[9, :] = 1e30
    x[10, 2] = 3.0e38
    x[11, :] = 1e-40              # fp32 subnormals
    xd, wd, sd = x.to(DEV), wq.to(DEV), s.to(DEV)
    L = _abi.lib()
    f32 = _abi.DTYPE_CODE[torch.float32]
    outs = []
    for nb in (L.cbq_w8a16_ws_bytes(M, N, K, 0, f32), _abi.WS_CTRL_BYTES):
        ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
        y = torch.empty(M, N, dtype=torch.float32, device=DEV)
        rc = L.cbq_w8a16_linear(_abi.ptr(xd), f32, _abi.ptr(wd), _abi.ptr(sd), None, None, 0,
                                None, M, N, K, _abi.ptr(ws), nb, _abi.ptr(y),
                                _abi.stream_handle(xd.device))
        _abi.check(rc, "w8a16 fp32")
        outs.append(y)
    torch.cuda.synchronize()
    yp, yg = outs
    assert torch.equal(torch.isnan(yp), torch.isnan(yg))
    assert torch.equal(torch.isinf(yp), torch.isinf(yg))
    fin = torch.isfinite(yg)
    assert torch.equal(torch.sign(yp[torch.isinf(yg)]), torch.sign(yg[torch.isinf(yg)]))
    xa = torch.where(torch.isfinite(xd), xd, torch.zeros((), device=DEV)).double().abs()
    bound = (xa @ wd.double().abs().t().contiguous()) * sd.double() * 2.0 ** -14 + 1e-30
    assert bool(((yp.double() - yg.double()).abs()[fin] <= bound[fin]).all())


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_empty_contraction(dt):
    """K == 0 (and M == 0 / N == 0): the reference's torch matmul gives
    zeros, times the scales, plus the bias."""
    for M, N in [(3, 40), (300, 1100)]:
        x = torch.empty(M, 0, dtype=dt, device=DEV)
        wq = torch.empty(N, 0, dtype=torch.int8, device=DEV)
        s = torch.rand(N, device=DEV).to(dt)
        b = torch.randn(N, device=DEV).to(dt)
        y = w8a16(x, wq, s, b)
        assert y.dtype == dt and tuple(y.shape) == (M, N)
        assert torch.equal(y, b.expand(M, N))
        assert bool((w8a16(x, wq, s) == 0).all())
    assert w8a16(torch.empty(0, 64, dtype=dt, device=DEV),
                 torch.zeros(8, 64, dtype=torch.int8, device=DEV),
                 torch.ones(8, dtype=dt, device=DEV)).shape == (0, 8)


def test_splitk_workspace_fallback():
    """A control-block-only workspace selects the no-split kernel; same
    results within fp32 accumulation order."""
    from cublade_amd import _abi
    M, K, N = 256, 2048, 1500
    x, wq, s, b, _, _ = make_case(M, K, N, torch.float16, 21, bias=True)
    xd, wd, sd, bd = x.to(DEV), wq.to(DEV), s.to(DEV), b.to(DEV)
    L = _abi.lib()
    assert L.cbq_w8a16_ws_bytes(M, N, K, 0, _abi.F16) > _abi.WS_CTRL_BYTES     # split-K shape
    y_split = w8a16(xd, wd, sd, bd)
    y_small = torch.empty_like(y_split)
    ws = torch.zeros(_abi.WS_CTRL_BYTES, dtype=torch.uint8, device=DEV)
    rc = L.cbq_w8a16_linear(_abi.ptr(xd), CODE_OF[torch.float16], _abi.ptr(wd), _abi.ptr(sd),
                            _abi.ptr(bd), None, 0, None, M, N, K, _abi.ptr(ws), ws.numel(),
                            _abi.ptr(y_small), _abi.stream_handle(xd.device))
    assert rc == 0
    torch.testing.assert_close(y_small.float(), y_split.float(), **TOL)
    ref = oracle_y(bits(x), oracle.F16, wq.numpy(), bits(s), bits(b), rows=np.array([0, 99, 255]))
    np.testing.assert_allclose(y_split.float().cpu().numpy()[[0, 99, 255]], ref, **TOL)


@pytest.mark.parametrize("M,K,N", [(1024, 2048, 1100), (1500, 2048, 700)])
def test_splitk_large_m_few_tiles(M, K, N):
    """M >= 1024 with fewer tiles than CUs takes the split-K path; rows
    against the oracle and the no-split kernel (control-block workspace)."""
    from cublade_amd import _abi
    L = _abi.lib()
    assert L.cbq_w8a16_ws_bytes(M, N, K, 0, _abi.BF16) > _abi.WS_CTRL_BYTES
    x, wq, s, b, _, _ = make_case(M, K, N, torch.bfloat16, M + N, bias=True)
    xd, wd, sd, bd = x.to(DEV), wq.to(DEV), s.to(DEV), b.to(DEV)
    y_split = w8a16(xd, wd, sd, bd)
    rows = np.array([0, 257, M // 2, M - 1])
    ref = oracle_y(bits(x), oracle.BF16, wq.numpy(), bits(s), bits(b), rows=rows)
    np.testing.assert_allclose(y_split.float().cpu().numpy()[rows], ref, **TOL)
    y_one = torch.empty_like(y_split)
    ws = torch.zeros(_abi.WS_CTRL_BYTES, dtype=torch.uint8, device=DEV)
    rc = L.cbq_w8a16_linear(_abi.ptr(xd), CODE_OF[torch.bfloat16], _abi.ptr(wd), _abi.ptr(sd),
                            _abi.ptr(bd), None, 0, None, M, N, K, _abi.ptr(ws), ws.numel(),
                            _abi.ptr(y_one), _abi.stream_handle(xd.device))
    assert rc == 0
    torch.testing.assert_close(y_split.float(), y_one.float(), **TOL)


@pytest.mark.parametrize("M,K,N,dt,n_out,path", [
    (128, 4096, 11008, torch.float16, 3, "128-row tiles, K in 4 ranges"),
    (512, 4096, 11008, torch.bfloat16, 0, "128-row tiles, whole"),
    (2137, 2048, 8192, torch.bfloat16, 20, "128-row tiles, 512 whole + the rest over 4 ranges"),
    (768, 4096, 11008, torch.float16, 33, "192-row tiles, whole (172 tiles in one wave)"),
    (139, 4096, 11008, torch.bfloat16, 1, "192-row tiles, K in 4 ranges, M tail"),
    (2211, 1024, 11008, torch.float16, 0, "192-row tiles, 512 whole + the rest over 4 ranges"),
    (1536, 4096, 11008, torch.bfloat16, 2, "256-row tiles, 256 whole + 2 over 16 ranges"),
    (3000, 1024, 5500, torch.float16, 18, "256-row tiles, 256 whole + 8 over 4 ranges, M and N tails"),
    (64, 11008, 4096, torch.float16, 2, "M <= 64 with long K: 128-row tiles over 11 ranges"),
    (32, 11008, 4096, torch.bfloat16, 1, "M = 32 with long K: 128-row tiles over 11 ranges"),
    (40, 16384, 1000, torch.bfloat16, 0, "M <= 64 with long K, N tail"),
    (256, 4096, 11008, torch.float16, 6, "128 x 128 tiles in one round (config 5, M = 256)"),
    (250, 2048, 14336, torch.bfloat16, 17, "128 x 128 tiles, M tail, two outlier chunks"),
    (96, 4096, 28672, torch.float16, 0, "128 x 128 tiles, one row of tiles"),
    (256, 3072, 14330, torch.float16, 1, "128 x 128 tiles, N tail (element stores)"),
    (383, 2048, 5000, torch.bfloat16, 3, "128 x 128 tiles, M and N tails"),
    (130, 2048, 28672, torch.float16, 0, "128-row tiles whole (224 tiles; 448 of 128 x 128 modelled slower)"),
    (320, 2048, 22016, torch.bfloat16, 2, "192-row tiles whole below 384 rows (no split)"),
])
def test_dma_plans(M, K, N, dt, n_out, path):
    """Each x-tile height (128, 192, 256 rows) and split plan of the MFMA tile
    path (whole tiles, all tiles over k-ranges, full waves whole plus a split
    tail, 128 x 128 tiles; the host's time model picks them per shape): sampled rows against
    the oracle, the full output against an fp32 product of the same operands
    (GPU matmul, independent of the kernel's tiling), and against the same
    call with a control-block workspace (no split)."""
    from cublade_amd import _abi
    print(f"[w8a16] {dt} M={M} K={K} N={N} outliers={n_out} ({path})", flush=True)
    rows = [0, M // 2 + 3, 2 * M // 3, M - 1]
    y = run_and_check(M, K, N, dt, seed=M + N, bias=True, n_out=n_out, rows=rows)
    x, wq, s, b, oc, w_out = make_case(M, K, N, dt, M + N, True, n_out)
    xd, wd, sd, bd = x.to(DEV), wq.to(DEV), s.to(DEV), b.to(DEV)
    ocd = torch.tensor(oc, dtype=torch.int64, device=DEV) if oc else None
    wod = w_out.to(DEV) if oc else None
    L = _abi.lib()
    y_one = torch.empty_like(y)
    ws = torch.zeros(_abi.WS_CTRL_BYTES, dtype=torch.uint8, device=DEV)
    rc = L.cbq_w8a16_linear(_abi.ptr(xd), CODE_OF[dt], _abi.ptr(wd), _abi.ptr(sd), _abi.ptr(bd),
                            None if ocd is None else _abi.ptr(ocd), n_out,
                            None if wod is None else _abi.ptr(wod), M, N, K, _abi.ptr(ws),
                            ws.numel(), _abi.ptr(y_one), _abi.stream_handle(xd.device))
    assert rc == 0
    torch.testing.assert_close(y.float(), y_one.float(), **TOL)
    wf = wd.float() * sd.float()[:, None]
    ref_full = xd.float() @ wf.t().contiguous() + bd.float()
    if oc:
        ref_full += xd.float()[:, ocd] @ wod.float().t().contiguous()
    torch.testing.assert_close(y.float(), ref_full, **TOL)


def test_mfma_bit_stability_across_calls():
    """Same inputs, same outputs, bit for bit (fixed accumulation order)."""
    x, wq, s, b, _, _ = make_case(256, 1024, 512, torch.float16, 8, bias=True)
    args = (x.to(DEV), wq.to(DEV), s.to(DEV), b.to(DEV))
    y0 = w8a16(*args)
    for _ in range(3):
        assert torch.equal(w8a16(*args), y0)


@pytest.mark.parametrize("M", [16, 256, 4096])
def test_config5_shapes(M):
    """x [M, 4096] N(0,1) with 6 feature columns at
    magnitude U(8, 20); W [11008, 4096] ~ N(0, 0.02) quantized per channel
    (fp16 scales)."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    g = torch.Generator().manual_seed(4)
    K, N = 4096, 11008
    x = torch.randn(M, K, generator=g)
    oc = torch.sort(torch.randperm(K, generator=g)[:6]).values
    mag = 8.0 + 12.0 * torch.rand(M, 6, generator=g)
    x[:, oc] = torch.sign(torch.randn(M, 6, generator=g)) * mag
    x = x.half()
    w = (0.02 * torch.randn(N, K, generator=g)).half()
    layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16).to(DEV)
    layer.quantize(w.to(DEV))
    assert layer.int8_weights.is_cuda and layer.scales.dtype == torch.float16
    y = layer(x.to(DEV))
    # every row at M = 16; else one row in every 64-row block (at a different
    # offset in each, so every x-tile and wave row position is sampled) plus
    # the first and last rows, against the oracle's exact accumulation
    rows = (np.arange(M) if M <= 16 else
            np.unique(np.r_[0, M - 1, [b * 64 + (b * 37 + 5) % 64 for b in range(M // 64)]])
            .astype(np.int64))
    ref = oracle_y(bits(x), oracle.F16, bits(layer.int8_weights), bits(layer.scales),
                   rows=rows)
    np.testing.assert_allclose(y.float().cpu().numpy()[rows], ref, **TOL)
    # whole output against a GPU fp32 product of the same operands
    wf = layer.int8_weights.float() * layer.scales.float()[:, None]
    ref_full = x.to(DEV).float() @ wf.t().contiguous()
    torch.testing.assert_close(y.float(), ref_full, **TOL)


@pytest.mark.parametrize("M", [16, 256, 4096])
def test_config5_activation_outliers(M):
    """BASELINE config 5 with the outlier threshold 6.0 applied the LLM.int8
    way (the layer's opt-in activation mode): the 6 feature columns of x at
    magnitude U(8, 20) become outlier columns, their weights stay fp16 for the
    side-GEMM and are zero in the INT8 copy; rows against the oracle (one in
    every 64-row block) and the whole output against an fp32 product."""
    from cublade_amd.benchmark import configs
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    x, w = configs.c5_w8a16(M)
    K, N = x.shape[1], w.shape[0]
    layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16, handle_outliers=True,
                                    outlier_threshold=6.0, outlier_mode="activation")
    layer.quantize(w.to(DEV), activations=x)
    oc = layer.outlier_cols.tolist()
    g = torch.Generator().manual_seed(4)
    torch.randn(M, K, generator=g)
    want = torch.sort(torch.randperm(K, generator=g)[:6]).values.tolist()
    assert oc == want, (oc, want)
    wq = layer.int8_weights
    assert int(wq[:, oc].abs().sum()) == 0
    xd = x.to(DEV)
    y = layer(xd)
    rows = (np.arange(M) if M <= 16 else
            np.unique(np.r_[0, M - 1, [b * 64 + (b * 29 + 3) % 64 for b in range(M // 64)]])
            .astype(np.int64))
    ref = oracle_y(bits(x), oracle.F16, bits(wq), bits(layer.scales), oc=oc,
                   w_out=bits(layer.outlier_weights), rows=rows)
    np.testing.assert_allclose(y.float().cpu().numpy()[rows], ref, **TOL)
    wf = wq.float() * layer.scales.float()[:, None]
    ref_full = xd.float() @ wf.t().contiguous() + \
        xd.float()[:, oc] @ layer.outlier_weights.float().t().contiguous()
    torch.testing.assert_close(y.float(), ref_full, **TOL)


def test_layer_outlier_mode_and_state_dict():
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    g = torch.Generator().manual_seed(12)
    K, N, M = 256, 128, 48
    w = 0.02 * torch.randn(N, K, generator=g)
    oc = [5, 77, 200]
    w[3, oc] = torch.tensor([7.5, -9.0, 6.5])
    w = w.half()
    layer = cuBladeW8A16LinearLayer(K, N, bias=True, dtype=torch.float16, handle_outliers=True)
    layer.quantize(w.to(DEV))
    assert layer.outlier_cols.tolist() == oc
    assert layer.int8_weights.shape == (N, K)
    assert torch.count_nonzero(layer.int8_weights[:, oc]).item() == 0
    layer.bias.data = (0.1 * torch.randn(N, generator=g)).half().to(DEV)
    layer.bias.requires_grad_(False)
    x = torch.randn(M, K, generator=g).half()
    x[:, oc] = 12.0
    y = layer(x.to(DEV))
    ref = oracle_y(bits(x), oracle.F16, bits(layer.int8_weights), bits(layer.scales),
                   bias=bits(layer.bias), oc=oc, w_out=bits(layer.outlier_weights))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, **TOL)
    # scales come from the normal columns only, as in the reference
    normal = [c for c in range(K) if c not in oc]
    amax = w.float()[:, normal].abs().amax(dim=1)
    inv = torch.tensor(127.0) / amax
    assert torch.equal(layer.scales.cpu(), (1.0 / inv).half())
    # CPU forward (reference CPU branch) agrees
    cpu = cuBladeW8A16LinearLayer(K, N, bias=True, dtype=torch.float16, handle_outliers=True)
    cpu.load_state_dict({k: v.cpu() for k, v in layer.state_dict().items()})
    y_cpu = cpu(x.float()).detach().float().numpy()
    np.testing.assert_allclose(y_cpu, ref, **TOL)
    # the saved layout is the reference's compact [N, K - n_out]; it loads
    # back and gives the same output
    sd = {k: v.cpu() for k, v in layer.state_dict().items()}
    assert tuple(sd["int8_weights"].shape) == (N, K - len(oc))
    assert torch.equal(sd["int8_weights"], layer.int8_weights.cpu()[:, normal])
    fresh = cuBladeW8A16LinearLayer(K, N, bias=True, dtype=torch.float16, handle_outliers=True)
    fresh.load_state_dict(sd)
    fresh = fresh.to(DEV)
    assert torch.equal(fresh.int8_weights, layer.int8_weights)
    assert torch.equal(fresh(x.to(DEV)), y)


def test_outlier_mode_unaligned_normal_width():
    """K - n_out not 16-byte aligned (4096 - 3 columns) works on the MFMA path;
    the reference rejects it (quantize_int8.cu:496-498)."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    g = torch.Generator().manual_seed(13)
    K, N, M = 4096, 512, 64
    w = 0.02 * torch.randn(N, K, generator=g)
    oc = [10, 2000, 4095]
    w[7, oc] = torch.tensor([8.0, -7.0, 9.5])
    layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16, handle_outliers=True)
    layer.quantize(w.half().to(DEV))
    assert layer.outlier_cols.tolist() == oc and layer.normal_cols.numel() == K - 3
    x = torch.randn(M, K, generator=g).half()
    y = layer(x.to(DEV))
    ref = oracle_y(bits(x), oracle.F16, bits(layer.int8_weights), bits(layer.scales), oc=oc,
                   w_out=bits(layer.outlier_weights))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, **TOL)


def test_quantize_model_mlp():
    from cublade_amd.quantization import cuBladeW8A16LinearLayer, quantize_model
    torch.manual_seed(42)
    model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 128), nn.ReLU(),
                          nn.Linear(128, 10)).half().to(DEV)
    x = torch.randn(32, 128).half().to(DEV)
    with torch.no_grad():
        y_fp = model(x).float()
    qm = quantize_model(model, "w8a16", exclude_modules=["4"], inplace=False)
    assert isinstance(qm[0], cuBladeW8A16LinearLayer) and isinstance(qm[2], cuBladeW8A16LinearLayer)
    assert isinstance(qm[4], nn.Linear)
    assert isinstance(model[0], nn.Linear)   # inplace=False left the original
    with torch.no_grad():
        y_q = qm(x).float()
    err = (y_q - y_fp).abs()
    assert err.max().item() < 0.05 and (err ** 2).mean().item() < 1e-4
    # layer 0 alone against the oracle
    with torch.no_grad():
        y0 = qm[0](x)
    ref = oracle_y(bits(x), oracle.F16, bits(qm[0].int8_weights), bits(qm[0].scales),
                   bias=bits(qm[0].bias.detach()))
    np.testing.assert_allclose(y0.float().cpu().numpy(), ref, **TOL)


def test_toy_flow_cpu_model():
    """The reference toy demo flow (examples/quantization/w8a16_toy_model.py):
    an fp32 MLP on the CPU is quantized (kernels on the GPU), buffers stay on
    the CPU, and the CPU forward follows the reference CPU branch."""
    from cublade_amd.quantization import quantize_model
    torch.manual_seed(42)
    model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 128), nn.ReLU(),
                          nn.Linear(128, 10))
    x = torch.randn(4, 128)
    with torch.no_grad():
        y_fp = model(x)
    qm = quantize_model(model, "w8a16", inplace=False)
    assert not qm[0].int8_weights.is_cuda and qm[0].scales.dtype == torch.float32
    with torch.no_grad():
        y_q = qm(x)
    assert ((y_q - y_fp) ** 2).mean().item() < 0.01 and (y_q - y_fp).abs().max().item() < 0.5
    # the same model on the GPU (fp32 activations: general path) agrees
    qg = qm.to(DEV)
    with torch.no_grad():
        y_g = qg(x.to(DEV)).cpu()
    torch.testing.assert_close(y_g, y_q, rtol=1e-4, atol=1e-4)


class _LlamaMLP(nn.Module):
    """LLaMA-style MLP block: down(silu(gate(x)) * up(x)), 4096 -> 11008 -> 4096."""

    def __init__(self, d=4096, h=11008, bias=False):
        super().__init__()
        self.gate_proj = nn.Linear(d, h, bias=bias)
        self.up_proj = nn.Linear(d, h, bias=bias)
        self.down_proj = nn.Linear(h, d, bias=bias)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


def _dequant_forward(block, x):
    """Forward of a block with each W8A16 layer replaced by an fp32 product
    x @ (wq * s)^T (+ bias) rounded once to fp16, i.e. the layer's contract;
    SiLU and the product run in fp16 as in the model."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer

    def lin(m, t):
        if isinstance(m, cuBladeW8A16LinearLayer):
            w = m.int8_weights.float() * m.scales.float()[:, None]
            b = None if m.bias is None else m.bias.float()
        else:
            w, b = m.weight.float(), None if m.bias is None else m.bias.float()
        y = t.float() @ w.t().contiguous()
        return (y if b is None else y + b).half()
    return lin(block.down_proj, torch.nn.functional.silu(lin(block.gate_proj, x)) *
               lin(block.up_proj, x))


def test_llama_mlp_stack_end_to_end():
    """quantize_model on two LLaMA-style MLP blocks (4096 -> 11008 -> 4096) in
    fp16 on the GPU, with a target filter and an exclude filter, one biased
    block, and forwards at M = 16 / 256 / 1024 (the streaming, split-K and
    tile kernels). Every W8A16 layer is checked at its real input inside the
    stack against an fp32 product rounded once (rtol/atol 1e-2), the chained
    output against the same computation in norm, and one layer against the
    oracle."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer, quantize_model
    torch.manual_seed(7)
    model = nn.Sequential(_LlamaMLP(), _LlamaMLP(bias=True))
    for p in model.parameters():
        nn.init.normal_(p, std=0.02)
    model = model.half().to(DEV)
    qm = quantize_model(model, "w8a16", target_modules=["proj"], exclude_modules=["1.down"],
                        inplace=False)
    for name in ("0.gate_proj", "0.up_proj", "0.down_proj", "1.gate_proj", "1.up_proj"):
        layer = qm.get_submodule(name)
        assert isinstance(layer, cuBladeW8A16LinearLayer), name
        assert layer.int8_weights.is_cuda and layer.scales.is_cuda
        assert layer.int8_weights.dtype == torch.int8 and layer.scales.dtype == torch.float16
    assert isinstance(qm.get_submodule("1.down_proj"), nn.Linear)
    assert qm[1].up_proj.bias is not None
    # every W8A16 layer's input and output inside the stack
    seen = []
    hooks = [m.register_forward_hook(lambda mod, inp, out: seen.append((mod, inp[0], out)))
             for m in qm.modules() if isinstance(m, cuBladeW8A16LinearLayer)]
    for M in (16, 256, 1024):
        x = torch.randn(M, 4096, device=DEV).half()
        seen.clear()
        with torch.no_grad():
            y = qm(x)
            y_fp = model(x).float()
            ref = _dequant_forward(qm[1], _dequant_forward(qm[0], x)).float()
        assert y.dtype == torch.float16 and tuple(y.shape) == (M, 4096)
        assert len(seen) == 5
        # each layer at its real input: fp32 product rounded once (north-star gate)
        for mod, inp, out in seen:
            w = mod.int8_weights.float() * mod.scales.float()[:, None]
            r = inp.float() @ w.t().contiguous()
            if mod.bias is not None:
                r = r + mod.bias.float()
            torch.testing.assert_close(out.float(), r.half().float(), **TOL)
        # the chained stack: ulp-level differences of the fp16 intermediates only
        assert ((y.float() - ref).norm() / ref.norm()).item() < 2e-3
        # quantization error of the whole stack next to the fp16 model: the
        # per-channel INT8 step is ~amax/127 ~ 4 sigma/127, i.e. ~0.9% relative
        # error per layer; five quantized layers compound to ~2.5%
        rel = ((y.float() - y_fp).norm() / y_fp.norm()).item()
        assert rel < 5e-2, rel
    for h in hooks:
        h.remove()
    # the first gate projection against the oracle on a few rows
    x = torch.randn(256, 4096).half()
    with torch.no_grad():
        y0 = qm[0].gate_proj(x.to(DEV))
    rows = np.array([0, 17, 255], np.int64)
    ref0 = oracle_y(bits(x), oracle.F16, bits(qm[0].gate_proj.int8_weights),
                    bits(qm[0].gate_proj.scales), rows=rows)
    np.testing.assert_allclose(y0.float().cpu().numpy()[rows], ref0, **TOL)
