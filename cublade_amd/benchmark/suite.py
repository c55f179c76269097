"""Benchmark suite over the BASELINE configurations (one GPU).

Each op is timed through the public API with HIP events, the Infinity Cache
flushed before every call, and reported as algorithmic bytes (or FLOPs) per
second and as a fraction of the MI355X roofline (8 TB/s HBM, 2.5 PFLOP/s
dense fp16 MFMA). Algorithmic bytes per op (N elements, C channels, G
groups): the op's minimum HBM traffic, 2N read + N written + 4 * scales for
every quant (x read once, codes and scales written), N + 4 * scales read +
2N written for every dequant. W8A16 and the dense GEMM: 2 * M * N * K
FLOPs (int8 GEMMs against the 5.0 POP/s dense int8 peak, the fp32-activation
W8A16 against the 157.3 TFLOP/s fp32 peak).

    python -m cublade_amd.benchmark.suite --configs c1,c2,c3,c3s,c4,c5,c5m,c5o,c5f32,f1,f3,fx,f4,f4s [--json out.json]

fx is a set of shapes off the configs (odd group sizes, few long rows,
narrow rows).
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys

import torch

from . import configs
from .core import (FP16_MFMA_PEAK_FLOP_S, HBM_PEAK_BYTES_S, I8_MFMA_PEAK_OP_S,
                   MallFlush, time_op)


def _rec(cfg, op, us, bytes_=None, flops=None):
    med = statistics.median(us)
    r = {"config": cfg, "op": op, "us_median": round(med, 2), "us_min": round(min(us), 2)}
    if bytes_ is not None:
        r["bytes"] = int(bytes_)
        r["gbs"] = round(bytes_ / med / 1e3, 1)
        r["hbm_frac"] = round(bytes_ / (med * 1e-6) / HBM_PEAK_BYTES_S, 4)
    if flops is not None:
        r["flops"] = int(flops)
        r["tflops"] = round(flops / med / 1e6, 2)
        r["mfma_frac"] = round(flops / (med * 1e-6) / FP16_MFMA_PEAK_FLOP_S, 4)
    return r


def run(selected, reps=20, warmup=3, flush_mode="clean"):
    from cublade_amd.quantization import (cuBladeW8A16LinearLayer, dequantize_tensor,
                                          quantize_tensor)
    dev = torch.device("cuda")
    flush = MallFlush(dev, mode=flush_mode)
    out = []

    def q_and_dq(cfg, x, qkw, q_bytes, dq_bytes, tag=""):
        qt = quantize_tensor(x, **qkw)
        out.append(_rec(cfg, "quant" + tag, time_op(lambda: quantize_tensor(x, **qkw), reps,
                                                     warmup, flush), q_bytes))
        out.append(_rec(cfg, "dequant" + tag, time_op(lambda: dequantize_tensor(qt), reps,
                                                      warmup, flush), dq_bytes))
        print(json.dumps(out[-2]), json.dumps(out[-1]), sep="\n", flush=True)

    if "c1" in selected:
        x = configs.c1_fp8_tensor().to(dev)
        n = x.numel()
        q_and_dq("c1", x, dict(dtype=torch.float8_e4m3fn, mode="tensor"),
                 2 * n + n + 4, n + 2 * n + 4)
        del x
    if "c2" in selected:
        x = configs.c2_int8_tensor().to(dev)
        n = x.numel()
        q_and_dq("c2", x, dict(dtype=torch.int8, mode="tensor"), 2 * n + n + 4,
                 n + 2 * n + 4)
        del x
    if "c3" in selected:
        x = configs.c3_int8_channel().to(dev)
        n, C, F = x.numel(), x.shape[0], x.shape[1]
        q_and_dq("c3", x, dict(dtype=torch.int8, mode="channel", ch_axis=0),
                 2 * n + n + 4 * C, n + 2 * n + 4 * C, "_axis0")
        q_and_dq("c3", x, dict(dtype=torch.int8, mode="channel", ch_axis=1),
                 2 * n + n + 4 * F, n + 2 * n + 4 * F, "_axis1")
        del x
    if "c3s" in selected:
        # config 3's weight cut to 8192 and 16384 rows (128 / 256 MiB): the
        # per-column (axis 1) quant then takes the one-launch path, x read once
        full = configs.c3_int8_channel()
        for rows in (8192, 16384):
            x = full[:rows].contiguous().to(dev)
            n, F = x.numel(), x.shape[1]
            q_and_dq("c3s", x, dict(dtype=torch.int8, mode="channel", ch_axis=1),
                     2 * n + n + 4 * F, n + 2 * n + 4 * F, f"_axis1_rows{rows}")
            del x
        del full
    if "c4" in selected:
        x = configs.c4_int8_group().to(dev)
        n = x.numel()
        G = n // 128
        q_and_dq("c4", x, dict(dtype=torch.int8, mode="group", group_size=128, ch_axis=-1),
                 2 * n + n + 4 * G, n + 2 * n + 4 * G)
        del x
    if "c5" in selected:
        # BASELINE config 5's M = 16 / 256 / 4096, plus M = 768 and 1536 (the
        # 192-row tiles in one wave, and 256-row tiles with a split last wave)
        for M in (16, 256, 768, 1536, 4096):
            x, w = configs.c5_w8a16(M)
            N, K = w.shape
            layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
            layer.quantize(w.to(dev))
            xd = x.to(dev)
            us = time_op(lambda: layer(xd), reps, warmup, flush)
            bytes_ = N * K + 2 * N + 2 * M * K + 2 * M * N
            r = _rec("c5", f"w8a16_m{M}", us, bytes_, 2.0 * M * N * K)
            out.append(r)
            print(json.dumps(r), flush=True)
            del layer, xd
    if "c5m" in selected:
        # the north star's M >= 1024 range of config 5's layer (every tile
        # plan the dispatcher uses there: whole waves, split tails)
        for M in (1024, 2048, 3072):
            x, w = configs.c5_w8a16(M)
            N, K = w.shape
            layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
            layer.quantize(w.to(dev))
            xd = x.to(dev)
            us = time_op(lambda: layer(xd), reps, warmup, flush)
            bytes_ = N * K + 2 * N + 2 * M * K + 2 * M * N
            r = _rec("c5m", f"w8a16_m{M}", us, bytes_, 2.0 * M * N * K)
            out.append(r)
            print(json.dumps(r), flush=True)
            del layer, xd
    if "c5o" in selected:
        # config 5 with its outlier threshold applied the LLM.int8 way (the
        # layer's opt-in activation mode): the 6 outlier features of x run
        # through the fp16 side-GEMM in the epilogue; the plain layer on the
        # same operands beside it gives the side-GEMM's cost
        for M in (16, 256, 4096):
            x, w = configs.c5_w8a16(M)
            N, K = w.shape
            lo = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16,
                                         handle_outliers=True, outlier_mode="activation")
            lo.quantize(w.to(dev), activations=x)
            xd = x.to(dev)
            us = time_op(lambda: lo(xd), reps, warmup, flush)
            bytes_ = N * K + 2 * N + 2 * M * K + 2 * M * N
            r = _rec("c5o", f"w8a16_outliers_m{M}", us, bytes_, 2.0 * M * N * K)
            r["n_out"] = int(lo.outlier_cols.numel())
            lp = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
            lp.quantize(w.to(dev))
            r["plain_us_median"] = round(statistics.median(time_op(lambda: lp(xd), reps, warmup,
                                                                   flush)), 2)
            out.append(r)
            print(json.dumps(r), flush=True)
            del lo, lp, xd
    if "c5f32" in selected:
        # The same layer with fp32 activations (an fp32 model under
        # quantize_model gets fp32 layers, utils.py:46). K % 64 == 0 and no
        # outlier columns: x as two bf16 planes on the matrix cores, twice
        # the MFMA work of the fp16 layer; mfma_frac counts both planes
        # against the 2.5 PFLOP/s bf16 peak.
        for M in (16, 256, 4096):
            x, w = configs.c5_w8a16(M)
            N, K = w.shape
            layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float32)
            layer.quantize(w.float().to(dev))
            xd = x.float().to(dev)
            us = time_op(lambda: layer(xd), max(3, reps // 4), warmup, flush)
            r = _rec("c5f32", f"w8a16_f32_m{M}", us, N * K + 4 * N + 4 * M * K + 4 * M * N,
                     2.0 * M * N * K)
            r["mfma_frac"] = round(2.0 * r["mfma_frac"], 4)
            out.append(r)
            print(json.dumps(r), flush=True)
            del layer, xd
    if "f1" in selected:
        # LLaMA-style MLP block, down(silu(gate(x)) * up(x)), 4096 -> 11008 ->
        # 4096, fp16, random N(0, 0.02) weights: W8A16 (quantize_model) next
        # to the fp16 block (PyTorch's own GEMMs).
        import torch.nn as nn
        from cublade_amd.quantization import quantize_model

        class Mlp(nn.Module):
            def __init__(self):
                super().__init__()
                self.gate_proj = nn.Linear(4096, 11008, bias=False)
                self.up_proj = nn.Linear(4096, 11008, bias=False)
                self.down_proj = nn.Linear(11008, 4096, bias=False)

            def forward(self, t):
                return self.down_proj(torch.nn.functional.silu(self.gate_proj(t)) * self.up_proj(t))

        g = torch.Generator().manual_seed(5)
        block = Mlp()
        with torch.no_grad():
            for prm in block.parameters():
                prm.copy_(0.02 * torch.randn(prm.shape, generator=g))
        block = block.half().to(dev).eval()
        qblock = quantize_model(block, "w8a16", inplace=False)
        for M in (16, 256, 4096):
            x = torch.randn(M, 4096, generator=g).half().to(dev)
            flops = 3 * 2.0 * M * 4096 * 11008
            with torch.no_grad():
                us_q = time_op(lambda: qblock(x), reps, warmup, flush)
                us_f = time_op(lambda: block(x), reps, warmup, flush)
            rq = _rec("f1", f"mlp_w8a16_m{M}", us_q, 3 * 4096 * 11008, flops)
            rf = _rec("f1", f"mlp_fp16_m{M}", us_f, 3 * 2 * 4096 * 11008, flops)
            rq["speedup_vs_fp16"] = round(statistics.median(us_f) / statistics.median(us_q), 3)
            out += [rq, rf]
            print(json.dumps(rq), json.dumps(rf), sep="\n", flush=True)
        # The M = 16 decode step captured in a HIP graph (torch.cuda.graph):
        # replays carry no per-call host work.
        x16 = torch.randn(16, 4096, generator=g).half().to(dev)
        flops = 3 * 2.0 * 16 * 4096 * 11008
        graph_us = {}
        for tag, blk in (("w8a16", qblock), ("fp16", block)):
            st = torch.cuda.Stream()
            with torch.no_grad(), torch.cuda.stream(st):
                for _ in range(3):
                    blk(x16)
            torch.cuda.synchronize()
            cg = torch.cuda.CUDAGraph()
            with torch.no_grad(), torch.cuda.graph(cg, stream=st):
                blk(x16)
            graph_us[tag] = time_op(cg.replay, reps, warmup, flush)
            del cg
        rq = _rec("f1", "mlp_w8a16_m16_graph", graph_us["w8a16"], 3 * 4096 * 11008, flops)
        rf = _rec("f1", "mlp_fp16_m16_graph", graph_us["fp16"], 3 * 2 * 4096 * 11008, flops)
        rq["speedup_vs_fp16"] = round(statistics.median(graph_us["fp16"]) /
                                      statistics.median(graph_us["w8a16"]), 3)
        out += [rq, rf]
        print(json.dumps(rq), json.dumps(rf), sep="\n", flush=True)
        del block, qblock
    if "f3" in selected:
        # Non-default axes in place: groups along axis 0 of config 4's tensor
        # and channels on the middle axis of config 3's tensor seen as
        # [7, 4096, 8192]. Each is timed next to the transposing route
        # (quantizers.py:122-132 / dequantizers.py:58-72): move the axis last,
        # contiguous copy, the same kernels, copy back.
        x = configs.c4_int8_group().to(dev)
        n = x.numel()
        G = n // 128
        qkw = dict(dtype=torch.int8, mode="group", group_size=128, ch_axis=0)
        q_and_dq("f3", x, qkw, 2 * n + n + 4 * G, n + 2 * n + 4 * G, "_group_axis0")
        lkw = dict(dtype=torch.int8, mode="group", group_size=128, ch_axis=-1)

        def group_via_copies():
            qt = quantize_tensor(x.movedim(0, -1).contiguous(), **lkw)
            return qt.data.movedim(-1, 0).contiguous()

        r = _rec("f3", "quant_group_axis0_via_copies",
                 time_op(group_via_copies, reps, warmup, flush), 2 * n + n + 4 * G)
        r["speedup_in_place"] = round(r["us_median"] / out[-2]["us_median"], 3)
        out.append(r)
        print(json.dumps(r), flush=True)
        del x
        x = configs.c3_int8_channel().to(dev).view(7, 4096, 8192)
        n, C = x.numel(), 4096
        q_and_dq("f3", x, dict(dtype=torch.int8, mode="channel", ch_axis=1),
                 2 * n + n + 4 * C, n + 2 * n + 4 * C, "_channel_axis1_3d")

        def channel_via_copies():
            qt = quantize_tensor(x.movedim(1, 0).contiguous(), dtype=torch.int8,
                                 mode="channel", ch_axis=0)
            return qt.data.movedim(0, 1).contiguous()

        r = _rec("f3", "quant_channel_axis1_3d_via_copies",
                 time_op(channel_via_copies, reps, warmup, flush), 2 * n + n + 4 * C)
        r["speedup_in_place"] = round(r["us_median"] / out[-2]["us_median"], 3)
        out.append(r)
        print(json.dumps(r), flush=True)
        del x
    if "fx" in selected:
        # Shapes off the configs, bf16 (random values; the bytes are the same
        # 2N + N + 4 * scales / N + 2N + 4 * scales as above): group sizes
        # that are not powers of two, rows of common LLM widths, few long
        # rows and narrow rows per channel.
        g = torch.Generator(device=dev).manual_seed(0)
        shapes = [
            ("_group56", (16384, 14336), dict(mode="group", group_size=56, ch_axis=1), 14336 // 56 * 16384),
            ("_group112", (16384, 14336), dict(mode="group", group_size=112, ch_axis=1),
             14336 // 112 * 16384),
            ("_group100", (16384, 14300), dict(mode="group", group_size=100, ch_axis=1),
             14300 // 100 * 16384),
            ("_channel_axis0_rows11008", (4096, 11008), dict(mode="channel", ch_axis=0), 4096),
            ("_channel_axis0_3d_64x1024x1024", (64, 1024, 1024), dict(mode="channel", ch_axis=0),
             64),
            ("_channel_axis0_256x262144", (256, 262144), dict(mode="channel", ch_axis=0), 256),
            ("_channel_axis1_262144x64", (262144, 64), dict(mode="channel", ch_axis=1), 64),
            ("_channel_axis1_16384x1000", (16384, 1000), dict(mode="channel", ch_axis=1), 1000),
            ("_channel_axis2_3d_256x512x512", (256, 512, 512), dict(mode="channel", ch_axis=2),
             512),
        ]
        for tag, shape, kw, nsc in shapes:
            x = torch.randn(*shape, device=dev, generator=g).bfloat16()
            n = x.numel()
            q_and_dq("fx", x, dict(dtype=torch.int8, **kw), 2 * n + n + 4 * nsc,
                     n + 2 * n + 4 * nsc, tag)
            del x
    if "f4" in selected:
        # Dense GEMM (wmma_gemm's replacement) at 8192^3: int8 -> int32 with B
        # as an [N, K] weight (read in place) and as [K, N] (transposed into
        # the workspace first, inside the timed call), uint8, fp16 -> fp32.
        # Next to PyTorch's own GEMMs (torch._int_mm, torch.matmul).
        from cublade_amd.bindings.hip.wmma import wmma_gemm
        M = N = K = 8192
        g = torch.Generator().manual_seed(6)
        flops = 2.0 * M * N * K
        a8 = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int16).to(torch.int8).to(dev)
        w8 = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int16).to(torch.int8).to(dev)
        b8 = w8.t().contiguous()
        cases = [("mm_i8_nk", lambda: wmma_gemm(a8, w8.t())),
                 ("mm_i8_kn", lambda: wmma_gemm(a8, b8)),
                 ("mm_u8_nk", lambda: wmma_gemm(a8.view(torch.uint8), w8.view(torch.uint8).t()))]
        try:
            torch._int_mm(a8[:32], w8.t()[:, :32].contiguous())
            cases.append(("torch_int_mm_i8", lambda: torch._int_mm(a8, w8.t())))
        except RuntimeError:
            pass
        for name, fn in cases:
            r = _rec("f4", name, time_op(fn, reps, warmup, flush), None, flops)
            r["tops"] = r.pop("tflops")
            r["mfma_frac"] = round(r["tops"] * 1e12 / I8_MFMA_PEAK_OP_S, 4)
            out.append(r)
            print(json.dumps(r), flush=True)
        del a8, w8, b8
        ah = torch.randn(M, K, generator=g).half().to(dev)
        wh = torch.randn(N, K, generator=g).half().to(dev)
        for name, fn in [("mm_f16_f32_nk", lambda: wmma_gemm(ah, wh.t())),
                         ("torch_matmul_f16", lambda: torch.matmul(ah, wh.t()))]:
            r = _rec("f4", name, time_op(fn, reps, warmup, flush), None, flops)
            out.append(r)
            print(json.dumps(r), flush=True)
        del ah, wh
    if "f4s" in selected:
        # The reference's own WMMA benchmark shapes (examples/kernels/
        # wmma_simple.py:137-150) up to 4096^3: few 256 x 256 tiles, K split.
        from cublade_amd.bindings.hip.wmma import wmma_gemm
        g = torch.Generator().manual_seed(7)
        for n in (512, 1024, 2048, 4096):
            fl = 2.0 * n ** 3
            a8 = torch.randint(-128, 128, (n, n), generator=g, dtype=torch.int16).to(torch.int8).to(dev)
            b8 = torch.randint(-128, 128, (n, n), generator=g, dtype=torch.int16).to(torch.int8).to(dev)
            ah = torch.randn(n, n, generator=g).half().to(dev)
            bh = torch.randn(n, n, generator=g).half().to(dev)
            for name, fn, i8 in [(f"mm_i8_kn_{n}", lambda: wmma_gemm(a8, b8), True),
                                 (f"torch_int_mm_i8_{n}", lambda: torch._int_mm(a8, b8), True),
                                 (f"mm_f16_f32_kn_{n}", lambda: wmma_gemm(ah, bh), False),
                                 (f"torch_matmul_f16_{n}", lambda: torch.matmul(ah, bh), False)]:
                r = _rec("f4s", name, time_op(fn, reps, warmup, flush), None, fl)
                if i8:
                    r["tops"] = r.pop("tflops")
                    r["mfma_frac"] = round(r["tops"] * 1e12 / I8_MFMA_PEAK_OP_S, 4)
                out.append(r)
                print(json.dumps(r), flush=True)
            del a8, b8, ah, bh
    torch.cuda.synchronize()
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="c1,c2,c3,c3s,c4,c5,c5m,c5o,c5f32,f1,f3,fx,f4,f4s")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--json", default=None)
    ap.add_argument("--flush", default="clean", choices=["clean", "dirty"])
    a = ap.parse_args(argv)
    res = run(set(a.configs.split(",")), a.reps, a.warmup, a.flush)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
