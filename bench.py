"""Benchmark of the MI355X quantization hot path (one GPU).

Workload: per-tensor symmetric INT8 of an fp16
[8192, 8192] tensor of 0.5 * Student-t(df=3) values, seed 1. One step is the
whole hot path over that tensor through the public API: quantize_tensor
(amax kernel + cast kernel) then dequantize_tensor (dequant kernel).

Timing: inputs resident in HBM. Before each timed phase a read-only sweep of
a 512 MiB buffer evicts the 256 MB Infinity Cache and the L2s (leaving clean
lines) and keeps the GPU busy while the host enqueues the phase; each phase
is timed with HIP events on its launch stream, the sweep outside the events.
value = algorithmic bytes of the K steps / summed phase time (GB/s).
Algorithmic bytes per step (N = 67,108,864): amax 2N + cast 2N + N + 4 +
dequant N + 2N + 4 = 536,870,920.

Roofline: the dequant kernel k_deq_tensor<int8, fp16>, the longest of the
three. Algorithmic bytes per launch: N codes read + 2N output bytes written +
4 scale bytes = 201,326,596 B. Its duration is measured live as the mean of
ROOF_LAUNCHES back-to-back launches between two HIP events on the launch
stream, after a cache sweep, each launch on its own copy of the codes and its
own output: ROOF_LAUNCHES x 201 MB = 2 GB of distinct buffers, so no launch
finds its codes, or the lines it writes, in the 256 MB Infinity Cache (the
steady-state HBM rate); peak 8 TB/s. traffic: HBM bytes per launch from
rocprofv3 FETCH_SIZE + WRITE_SIZE runs, read from
profiles/dequant_int8_c2_traffic.json when present (null otherwise).

Extra keys: per-phase GB/s, the W8A16 linear at M = 4096 (BASELINE
configs[4]) in TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak, and
copy_ceiling: a plain device-to-device copy moving the roofline kernel's
byte count, timed the same way (distinct buffers per launch), the
achievable HBM rate next to the 8 TB/s spec.

cpu_baseline: the C oracle (test infrastructure, single thread) on the first
8,388,608 elements of the same tensor, repeated for about 10 s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import dataclasses
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
ROOF_LAUNCHES = 10
TRAFFIC_FILE = ROOT / "profiles" / "dequant_int8_c2_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-w8a16", action="store_true", help="skip the W8A16 extra")
    ap.add_argument("--flush", default="clean", choices=["clean", "dirty"])
    return ap.parse_args()


def cpu_baseline(x_cpu):
    import numpy as np
    import torch

    import oracle

    sample = x_cpu.reshape(-1)[: 8 * 1024 * 1024].contiguous()
    xb = sample.view(torch.int16).numpy().view(np.uint16)
    n = xb.size
    t_total, reps = 0.0, 0
    while t_total < 10.0 and reps < 500:
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


def timed_rotation(torch, stream, flush, ev, fns):
    """Mean launch time (us) of fns[0..] run back to back between two HIP
    events after a cache sweep; the best of 3 sweeps."""
    outs = [f() for f in fns]      # every output block cached by the allocator
    del outs
    runs = []
    for _ in range(3):
        flush()
        a, b = ev(), ev()
        a.record(stream)
        outs = [f() for f in fns]
        b.record(stream)
        runs.append((a, b))
        del outs
    torch.cuda.synchronize()
    return min(a.elapsed_time(b) for a, b in runs) * 1e3 / len(fns)


def copy_ceiling(torch, dev, stream, flush, ev):
    """Achievable HBM rate next to the 8 TB/s spec: the runtime's
    device-to-device copy moving the roofline kernel's byte count (half
    read, half written), over ROOF_LAUNCHES distinct buffer pairs."""
    nbytes = (BYTES_DEQ - 4) // 2
    pairs = [(torch.ones(nbytes, dtype=torch.uint8, device=dev),
              torch.empty(nbytes, dtype=torch.uint8, device=dev)) for _ in range(ROOF_LAUNCHES)]
    us = timed_rotation(torch, stream, flush, ev,
                        [lambda s=s_, d=d_: d.copy_(s) for s_, d_ in pairs])
    del pairs
    gbs = 2 * nbytes / (us * 1e-6) / 1e9
    return {"what": f"torch copy_ of {nbytes} B (device to device), {ROOF_LAUNCHES} buffer pairs",
            "bytes_moved": 2 * nbytes, "avg_launch_us": round(us, 2), "gbs": round(gbs, 2),
            "frac": round(gbs * 1e9 / HBM_PEAK, 4)}


def w8a16_extra(torch, reps):
    from cublade_amd.benchmark import configs
    from cublade_amd.benchmark.core import MallFlush, time_op
    from cublade_amd.quantization import cuBladeW8A16LinearLayer

    dev = torch.device("cuda")
    x, w = configs.c5_w8a16(4096)
    N, K = w.shape
    layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
    layer.quantize(w.to(dev))
    xd = x.to(dev)
    us = time_op(lambda: layer(xd), reps, 2, MallFlush(dev))
    us_med = sorted(us)[len(us) // 2]
    flops = 2.0 * 4096 * N * K
    return {"w8a16_m4096_us": round(us_med, 2),
            "w8a16_m4096_tflops": round(flops / us_med / 1e6, 2),
            "w8a16_m4096_mfma_frac": round(flops / (us_med * 1e-6) / FP16_PEAK, 4)}


def load_traffic():
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        return float(d["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the multi-GPU layout is described in DESIGN.md)"}))
        sys.exit(2)
    import torch

    from cublade_amd import _abi
    from cublade_amd.benchmark import configs
    from cublade_amd.benchmark.core import MallFlush
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor

    _abi.lib()
    dev = torch.device("cuda:0")
    x_cpu = configs.c2_int8_tensor()
    x = x_cpu.to(dev)
    flush = MallFlush(dev, mode=args.flush)
    stream = torch.cuda.current_stream(dev)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def step(t_q, t_d):
        flush()
        e0, e1, e2, e3 = ev(), ev(), ev(), ev()
        e0.record(stream)
        qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
        e1.record(stream)
        flush()
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
    quant_us = sum(q_ms) / len(q_ms) * 1e3
    deq_us = sum(d_ms) / len(d_ms) * 1e3

    # roofline kernel: back-to-back dequant launches after one sweep, each on
    # its own copy of the codes (2 GB of distinct inputs and outputs)
    qts = [dataclasses.replace(qt, data=qt.data.clone()) for _ in range(ROOF_LAUNCHES)]
    roof_us = timed_rotation(torch, stream, flush, ev,
                             [lambda t=t: dequantize_tensor(t) for t in qts])
    del qts
    achieved = BYTES_DEQ / (roof_us * 1e-6) / 1e9
    copy = copy_ceiling(torch, dev, stream, flush, ev)

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
                   "cache_sweep": args.flush},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved * 1e9 / HBM_PEAK, 4),
                     "traffic": load_traffic(), "kernel": "k_deq_tensor<int8, fp16>",
                     "bytes_per_launch": BYTES_DEQ, "avg_launch_us": round(roof_us, 2)},
        "copy_ceiling": copy,
        "phases": {"quant_us": round(quant_us, 2),
                   "quant_gbs": round((BYTES_AMAX + BYTES_CAST) / quant_us / 1e3, 2),
                   "dequant_us": round(deq_us, 2),
                   "dequant_gbs": round(BYTES_DEQ / deq_us / 1e3, 2)},
        "wall_s_incl_sweeps": round(wall, 3),
    }
    if not args.no_w8a16:
        out.update(w8a16_extra(torch, max(3, args.steps // 2)))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x_cpu)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
