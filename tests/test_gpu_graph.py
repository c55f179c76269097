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


@pytest.mark.parametrize("M", [16, 256, 4096])
def test_graph_w8a16_layer(M):
    """The W8A16 layer at a decode shape (weight streaming), at M = 256
    (split-K: fp32 partials in the workspace, reused by every replay) and at
    M = 4096 (256-row MFMA tiles, whose kernel keeps a few spilled registers
    in scratch memory)."""
    from cublade_amd.quantization import cuBladeW8A16LinearLayer
    N, K = 4096, 2048
    g0 = torch.Generator().manual_seed(M)
    layer = cuBladeW8A16LinearLayer(K, N, bias=True, dtype=torch.float16)
    layer.quantize((0.02 * torch.randn(N, K, generator=g0)).half().to(DEV))
    with torch.no_grad():
        layer.bias.copy_((0.1 * torch.randn(N, generator=g0)).half())
    layer = layer.to(DEV)   # the bias parameter too: a captured call copies nothing from the host
    x = torch.randn(M, K, generator=g0).half().to(DEV)
    s = torch.cuda.Stream()
    with torch.no_grad():
        fn = lambda: layer(x)
        g, out = _capture(fn, s)
        _check_replays(x, lambda i: torch.randn(M, K, generator=torch.Generator().manual_seed(100 + i))
                       .half().to(DEV), fn, g, out)


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
