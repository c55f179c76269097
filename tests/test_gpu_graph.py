"""HIP graph capture of the hot path (torch.cuda.graph over the C ABI).

The entry points allocate nothing and never synchronize, so a decode loop
can capture them and replay without per-call host work. Each test warms up
on the capture stream (the per-stream workspace is allocated then, outside
the capture), captures one call, and replays it three times with new input
contents copied in eagerly between replays; every replay must equal the
eager call on the same input bit for bit (same kernels, same order).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _capture(fn, stream):
    """Warm up fn on `stream`, then capture one call into a graph."""
    with torch.cuda.stream(stream):
        for _ in range(2):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _check_replays(static_in, make_input, fn, g, out, n=3):
    for seed in range(n):
        fresh = make_input(seed)
        static_in.copy_(fresh)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = fn()
        torch.cuda.synchronize()
        for o, w in zip(out if isinstance(out, tuple) else (out,),
                        want if isinstance(want, tuple) else (want,)):
            assert torch.equal(o.view(torch.uint8) if o.dtype.itemsize == 1 else o,
                               w.view(torch.uint8) if w.dtype.itemsize == 1 else w), f"replay {seed}"


@pytest.mark.parametrize("M,dt,N,K", [(16, torch.float16, 4096, 2048), (256, torch.float16, 4096, 2048),
                                      (4096, torch.float16, 4096, 2048), (256, torch.float32, 4096, 2048),
                                      (256, torch.bfloat16, 11008, 4096)])
def test_graph_w8a16_layer(M, dt, N, K):
    """The W8A16 layer at a decode shape (weight streaming), at M = 256
    (split-K: fp32 partials in the workspace, reused by every replay), at
    M = 4096 (256-row MFMA tiles, whose kernel keeps a few spilled registers
    in scratch memory), with fp32 activations at M = 256 (three launches:
    the bf16 planes of x and the partial planes in the workspace), and at
    config 5's M = 256 (one round of 128 x 128 tiles, no workspace)."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    g0 = torch.Generator().manual_seed(M)
    layer = cuBladeW8A16LinearLayer(K, N, bias=True, dtype=dt)
    layer.quantize((0.02 * torch.randn(N, K, generator=g0)).to(dt).to(DEV))
    with torch.no_grad():
        layer.bias.copy_((0.1 * torch.randn(N, generator=g0)).to(dt))
    layer = layer.to(DEV)   # the bias parameter too: a captured call copies nothing from the host
    x = torch.randn(M, K, generator=g0).to(dt).to(DEV)
    s = torch.cuda.Stream()
    with torch.no_grad():
        fn = lambda: layer(x)
        g, out = _capture(fn, s)
        _check_replays(x, lambda i: torch.randn(M, K, generator=torch.Generator().manual_seed(100 + i))
                       .to(dt).to(DEV), fn, g, out)


def test_graph_quant_dequant_per_tensor():
    """Per-tensor INT8 quant (amax partials in the workspace) then dequant."""
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    n = 1 << 22
    x = torch.randn(n, generator=torch.Generator().manual_seed(1)).half().to(DEV)

    def fn():
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        return qt.data, qt.scale, dequantize_tensor(qt)

    g, out = _capture(fn, torch.cuda.Stream())
    _check_replays(x, lambda i: (3.0 * i + 1.0) * torch.randn(n, generator=torch.Generator()
                                                              .manual_seed(10 + i)).half().to(DEV),
                   fn, g, out)


def test_graph_per_column_one_launch_and_per_tensor():
    """The one-launch per-column quant (two grid-wide exchanges through the
    workspace's control block) and the one-launch per-tensor quant, sharing
    that control block, captured in one graph: every replay's tags follow
    the generation left in memory by the one before."""
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    x = (0.02 * torch.randn(2048, 8192, generator=torch.Generator().manual_seed(4))).bfloat16().to(DEV)

    def fn():
        qc = quantize_tensor(x, dtype=torch.int8, mode="channel", ch_axis=1)
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        return qc.data, qc.scale, qt.data, qt.scale, dequantize_tensor(qc)

    g, out = _capture(fn, torch.cuda.Stream())
    _check_replays(x, lambda i: ((0.5 + i) * torch.randn(2048, 8192, generator=torch.Generator()
                                                         .manual_seed(40 + i))).bfloat16().to(DEV),
                   fn, g, out)


def test_graph_group_and_fp8():
    """Per-group INT8 (G = 128) and per-tensor FP8 in one graph."""
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    x = torch.randn(512, 1024, generator=torch.Generator().manual_seed(2)).bfloat16().to(DEV)

    def fn():
        qg = quantize_tensor(x, dtype=torch.int8, mode="group", group_size=128, ch_axis=-1)
        qf = quantize_tensor(x, dtype=torch.float8_e4m3fn, mode="tensor")
        return qg.data, qg.scale, qf.data, qf.scale, dequantize_tensor(qg), dequantize_tensor(qf)

    g, out = _capture(fn, torch.cuda.Stream())
    _check_replays(x, lambda i: torch.randn(512, 1024, generator=torch.Generator()
                                            .manual_seed(20 + i)).bfloat16().to(DEV), fn, g, out)


def test_graph_workspace_survives_growth():
    """Two graphs captured on one stream whose second warm-up grows that
    stream's workspace: the first graph's workspace (its per-tensor control
    block) stays allocated, and its replays stay exact while the caching
    allocator hands out fresh memory in between. Growing inside a capture
    raises instead of allocating."""
    from cublade_amd import _abi
    from cublade_amd.quantization import cuBladeW8A16LinearLayer, quantize_tensor
    s = torch.cuda.Stream()
    n = 1 << 22
    x = torch.randn(n, generator=torch.Generator().manual_seed(3)).half().to(DEV)

    def quant():
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        return qt.data, qt.scale

    g1, out1 = _capture(quant, s)
    with torch.cuda.stream(s):
        ws1 = _abi.workspace(x.device, 0)
    ptr1, size1 = ws1.data_ptr(), ws1.numel()
    del ws1
    # M = 128, N = 11008: split-K partials, a workspace far larger than size1
    N, K, M = 11008, 4096, 128
    layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
    layer.quantize((0.02 * torch.randn(N, K, generator=torch.Generator().manual_seed(4)))
                   .half().to(DEV))
    xa = torch.randn(M, K, generator=torch.Generator().manual_seed(5)).half().to(DEV)
    with torch.no_grad():
        g2, out2 = _capture(lambda: layer(xa), s)
    with torch.cuda.stream(s):
        ws2 = _abi.workspace(x.device, 0)
    assert ws2.numel() > size1 and ws2.data_ptr() != ptr1
    assert any(t.data_ptr() == ptr1 for t in _abi._ws_retired)
    # fresh allocations that would reuse a freed workspace
    junk = [torch.full((size1,), 0x5A, dtype=torch.uint8, device=DEV) for _ in range(4)]
    _check_replays(x, lambda i: (2.0 + i) * torch.randn(n, generator=torch.Generator()
                                                        .manual_seed(30 + i)).half().to(DEV),
                   quant, g1, out1)
    with torch.no_grad():
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, layer(xa))
    assert all(bool((j == 0x5A).all()) for j in junk)
    # a shape that needs more workspace than the capture stream holds
    big = cuBladeW8A16LinearLayer(K, 4 * N, bias=False, dtype=torch.float16)
    big.quantize(torch.zeros(4 * N, K, dtype=torch.float16, device=DEV))
    xb = torch.randn(1536, K, generator=torch.Generator().manual_seed(6)).half().to(DEV)
    need = _abi.lib().cbq_w8a16_ws_bytes(1536, 4 * N, K, 0, _abi.F16)
    if need > ws2.numel():
        g3 = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="during graph capture"):
            with torch.no_grad(), torch.cuda.graph(g3, stream=s):
                big(xb)
    torch.cuda.synchronize()
