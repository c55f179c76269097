"""Benchmark of the MI355X quantization hot path (one GPU).

Workload: per-tensor symmetric INT8 of an fp16
[8192, 8192] tensor of 0.5 * Student-t(df=3) values, seed 1. One step is the
whole hot path over that tensor: quantize_tensor (amax kernel + cast kernel)
then dequantize_tensor (dequant kernel), through the public API.

Timing: inputs resident in HBM; before each timed phase a 512 MiB
read-modify-write of a scratch buffer evicts the 256 MB Infinity Cache (and
keeps the GPU busy while the host enqueues the phase); each phase is timed
with HIP events on the launch stream and the flush is outside the events.
value = algorithmic bytes of the K steps / summed phase time.

Roofline: the dequant kernel (one launch per dequantize_tensor call),
algorithmic bytes per launch = 67,108,864 codes read + 134,217,728 output
bytes written + 4 scale bytes = 201,326,596 B, over its event-timed
duration; peak 8 TB/s. traffic: HBM bytes per launch measured separately
with rocprofv3 FETCH_SIZE / WRITE_SIZE (see profiles/), passed in via
--traffic-bytes or null.

Also reported (extra keys): each phase's GB/s, and the W8A16 linear at
M = 4096 in TFLOP/s against the 2.5 PFLOP/s dense
fp16 MFMA peak.

cpu_baseline: the C oracle (test infrastructure, single thread) on the
first 8,388,608 elements of the same tensor, repeated for about 10 s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
os.environ.setdefault("CUBLADE_SKIP_WARMUP", "1")

HBM_PEAK = 8.0e12
FP16_PEAK = 2.5e15
N_ELEM = 8192 * 8192
BYTES_AMAX = 2 * N_ELEM
BYTES_CAST = 2 * N_ELEM + N_ELEM + 4
BYTES_DEQ = N_ELEM + 2 * N_ELEM + 4
BYTES_STEP = BYTES_AMAX + BYTES_CAST + BYTES_DEQ


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-w8a16", action="store_true", help="skip the W8A16 extra")
    ap.add_argument("--traffic-bytes", type=float, default=None,
                    help="rocprofv3-measured HBM bytes per dequant launch")
    return ap.parse_args()


def make_input(torch):
    g = torch.Generator().manual_seed(1)
    shape = (8192, 8192)
    z = torch.randn(*shape, generator=g)
    c = [torch.randn(*shape, generator=g) for _ in range(3)]
    t = z / torch.sqrt((c[0] ** 2 + c[1] ** 2 + c[2] ** 2) / 3)
    x = (0.5 * t).half()
    assert torch.isfinite(x).all()
    return x


def cpu_baseline(x_cpu):
    import numpy as np
    import oracle

    sample = x_cpu.reshape(-1)[: 8 * 1024 * 1024].contiguous()
    xb = sample.view(__import__("torch").int16).numpy().view(np.uint16)
    n = xb.size
    t_total, reps = 0.0, 0
    while t_total < 10.0 and reps < 50:
        t0 = time.perf_counter()
        q, s = oracle.quant_int8_tensor(xb, oracle.F16)
        oracle.dequant_int8_tensor(q, s, oracle.F16)
        t_total += time.perf_counter() - t0
        reps += 1
    per_elem = 2 + 3 + 3
    return {
        "value": round(per_elem * n * reps / t_total / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"C oracle (oracle/cbq_oracle.c, 1 thread) quant+dequant of the first "
                  f"{n} elements of the workload tensor, {reps} reps, {t_total:.1f} s; "
                  f"host {os.cpu_count()} logical CPUs",
    }


def w8a16_extra(torch, steps):
    from cublade_amd.bindings.hip import w8a16_linear

    g = torch.Generator().manual_seed(4)
    M, K, N = 4096, 4096, 11008
    x = torch.randn(M, K, generator=g)
    oc = torch.sort(torch.randperm(K, generator=g)[:6]).values
    x[:, oc] = torch.sign(torch.randn(M, 6, generator=g)) * (8 + 12 * torch.rand(M, 6, generator=g))
    dev = torch.device("cuda")
    x = x.half().to(dev)
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    s = (torch.rand(N, generator=g) * 1e-3).half().to(dev)
    y = w8a16_linear(x, wq, s)
    for _ in range(3):
        y = w8a16_linear(x, wq, s)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(steps):
        y = w8a16_linear(x, wq, s)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / steps
    flops = 2.0 * M * N * K
    del y
    return {"w8a16_m4096_ms": round(ms, 4), "w8a16_m4096_tflops": round(flops / ms / 1e9, 2),
            "w8a16_m4096_mfma_frac": round(flops / (ms * 1e-3) / FP16_PEAK, 4)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the multi-GPU layout is described in DESIGN.md)"}))
        sys.exit(2)
    import torch

    from cublade_amd import _abi
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor

    _abi.lib()
    dev = torch.device("cuda:0")
    x_cpu = make_input(torch)
    x = x_cpu.to(dev)
    flush = torch.zeros(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step(t_q, t_d):
        flush.add_(1)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e2 = torch.cuda.Event(enable_timing=True)
        e3 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        e1.record(stream)
        flush.add_(1)
        e2.record(stream)
        y = dequantize_tensor(qt)
        e3.record(stream)
        t_q.append((e0, e1))
        t_d.append((e2, e3))
        return qt, y

    for _ in range(args.warmup):
        step([], [])
    torch.cuda.synchronize()

    tq, td = [], []
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for _ in range(args.steps):
        qt, y = step(tq, td)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    q_ms = [a.elapsed_time(b) for a, b in tq]
    d_ms = [a.elapsed_time(b) for a, b in td]
    sum_s = (sum(q_ms) + sum(d_ms)) / 1e3
    value = BYTES_STEP * args.steps / sum_s / 1e9
    deq_avg_s = sum(d_ms) / len(d_ms) / 1e3
    deq_gbs = BYTES_DEQ / deq_avg_s / 1e9
    quant_gbs = (BYTES_AMAX + BYTES_CAST) / (sum(q_ms) / len(q_ms) / 1e3) / 1e9

    out = {
        "metric": "quant/dequant HBM GB/s (% of peak) at 1 MI355X; W8A16 TFLOPS at M=4096",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sum_s * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (BASELINE configs[1] recipe, seed 1)",
        "config": {"workload": "INT8 per-tensor quantize_tensor + dequantize_tensor, fp16 "
                               "[8192, 8192] 0.5*t(df=3), seed 1 (BASELINE configs[1])",
                   "hbm_frac": round(value * 1e9 / HBM_PEAK, 4),
                   "mall_flushed": True},
        "roofline": {"bound": "hbm", "achieved": round(deq_gbs, 2), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(deq_gbs * 1e9 / HBM_PEAK, 4),
                     "traffic": args.traffic_bytes, "kernel": "k_deq_tensor<int8, fp16>",
                     "bytes_per_launch": BYTES_DEQ,
                     "avg_launch_us": round(deq_avg_s * 1e6, 2)},
        "phases": {"quant_gbs": round(quant_gbs, 2), "quant_us": round(sum(q_ms) / len(q_ms) * 1e3, 2),
                   "dequant_gbs": round(deq_gbs, 2), "dequant_us": round(deq_avg_s * 1e6, 2)},
        "wall_s_incl_flush": round(wall, 3),
    }
    if not args.no_w8a16:
        out.update(w8a16_extra(torch, max(3, args.steps // 4)))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x_cpu)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
