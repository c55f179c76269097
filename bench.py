"""Benchmark of the MI355X quantization hot path (one GPU).

Workload: per-tensor symmetric INT8 of an fp16
[8192, 8192] tensor of 0.5 * Student-t(df=3) values, seed 1. One step is the
whole hot path over that tensor through the public API: quantize_tensor (one
launch of k_quant_tensor_1pass) then dequantize_tensor (k_deq_tensor).

Timing: inputs resident in HBM. Before each timed phase a sweep of a 512 MiB
buffer evicts the 256 MB Infinity Cache and the L2s and keeps the GPU busy
while the host enqueues the phase; each phase is timed with HIP events on its
launch stream, the sweep outside the events. The headline uses a read-only
sweep (clean cache lines); the same steps are then repeated after a write
sweep (every line dirty, the worst case after a large producer) and reported
next to it as "dirty".

Algorithmic bytes (N = 67,108,864 elements): each op's minimum HBM traffic,
quant 2N read + N codes + 4 scale bytes, dequant N + 4 read + 2N written;
6N + 8 = 402,653,192 bytes per step. value = those bytes of the K steps /
the summed phase time (GB/s).

Roofline: every kernel of the step is timed live as the mean of ROOF_LAUNCHES
back-to-back launches between two HIP events on the launch stream, after one
cache sweep, each launch on its own input and output buffers (about 2 GB of
distinct buffers per kernel, so no launch finds its data in the 256 MB
Infinity Cache); `roofline` reports the longest one (the quant kernel),
`kernels` all of them. achieved = the kernel's algorithmic bytes per launch /
its mean launch time; peak 8 TB/s. traffic: HBM bytes per launch from
rocprofv3 FETCH_SIZE and WRITE_SIZE runs of this script, calibrated on a
256 MiB device copy (profiles/quant_int8_c2_traffic.json; null if absent).

Extras, timed in the same run (HIP events around each op after a clean
sweep, median of EXTRA_REPS): every other BASELINE config (C1 FP8 per
tensor, C3 per channel on both axes, C4 per group, W8A16 at M = 16, 256 and
4096, each next to an fp16 F.linear of the dequantized weight). Their inputs follow the configs' distributions but are drawn on the
GPU (torch's device generator), which makes no difference to the timing of
these data-independent kernels; the parity tests use the CPU-seeded recipes.

cpu_baseline: the torch CPU restatement of the same formulas
(oracle/torch_cpu.py) on the full workload tensor, torch.set_num_threads(
os.cpu_count()), one warm-up then the median of CPU_REPS quant + dequant
steps, with its codes and outputs compared to the GPU's.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
os.environ.setdefault("CUBLADE_SKIP_WARMUP", "1")

HBM_PEAK = 8.0e12
FP16_PEAK = 2.5e15
N_ELEM = 8192 * 8192
BYTES_QUANT = 2 * N_ELEM + N_ELEM + 4
BYTES_DEQ = N_ELEM + 4 + 2 * N_ELEM
BYTES_STEP = BYTES_QUANT + BYTES_DEQ
ROOF_LAUNCHES = 10
EXTRA_REPS = 10
CPU_REPS = 3
TRAFFIC_FILE = ROOT / "profiles" / "quant_int8_c2_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip the other configs")
    ap.add_argument("--no-w8a16", action="store_true", help="skip the W8A16 extras")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(x_cpu, q_gpu, y_gpu):
    import numpy as np
    import torch

    from oracle import torch_cpu

    torch.set_num_threads(os.cpu_count() or 1)
    times = []
    for r in range(CPU_REPS + 1):
        t0 = time.perf_counter()
        q, s = torch_cpu.quant_tensor(x_cpu, torch.int8)
        y = torch_cpu.dequant_tensor(q, s, torch.float16)
        dt = time.perf_counter() - t0
        if r:
            times.append(dt)
    med = statistics.median(times)
    same = bool(torch.equal(q, q_gpu.cpu())) and bool(
        np.array_equal(y.view(torch.int16).numpy(), y_gpu.cpu().view(torch.int16).numpy()))
    return {
        "value": round(BYTES_STEP / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"the full workload tensor ({N_ELEM} fp16 elements): torch CPU restatement "
                  f"(oracle/torch_cpu.py) of quant + dequant, median of {CPU_REPS} steps after "
                  f"1 warm-up, {med * 1e3:.1f} ms per step; os.cpu_count() = {os.cpu_count()}, "
                  f"torch threads = {torch.get_num_threads()}, CPU: {cpu_model()}; codes and "
                  f"outputs bit-identical to the GPU's: {same}",
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
    device-to-device copy moving the dequant kernel's byte count (half read,
    half written), over ROOF_LAUNCHES distinct buffer pairs."""
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


def _rate(bytes_, us):
    return {"us": round(us, 2), "gbs": round(bytes_ / us / 1e3, 1),
            "hbm_frac": round(bytes_ / (us * 1e-6) / HBM_PEAK, 4)}


def extras(torch, dev, no_w8a16):
    """Every other BASELINE config through the public API, op-level HIP
    event times after a clean sweep (median of EXTRA_REPS)."""
    from cublade_amd.benchmark import configs
    from cublade_amd.benchmark.core import MallFlush, time_op
    from cublade_amd.quantization import (cuBladeW8A16LinearLayer, dequantize_tensor,
                                          quantize_tensor)

    flush = MallFlush(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    out = {}

    def qdq(name, x, qkw, q_bytes, dq_bytes):
        qt = quantize_tensor(x, **qkw)
        tq = statistics.median(time_op(lambda: quantize_tensor(x, **qkw), EXTRA_REPS, 2, flush))
        td = statistics.median(time_op(lambda: dequantize_tensor(qt), EXTRA_REPS, 2, flush))
        out[name] = {"quant": _rate(q_bytes, tq), "dequant": _rate(dq_bytes, td)}
        print(f"[bench] {name}: quant {tq:.1f} us, dequant {td:.1f} us", file=sys.stderr,
              flush=True)

    x = torch.randn(4096, 4096, device=dev, generator=g).bfloat16()
    n = x.numel()
    qdq("c1_fp8_tensor_bf16_4096x4096", x, dict(dtype=torch.float8_e4m3fn, mode="tensor"),
        3 * n + 4, 3 * n + 4)
    del x
    x = 0.02 * torch.randn(28672, 8192, device=dev, generator=g)
    cols = torch.randperm(8192, device=dev, generator=g)[:8]
    x[:, cols] *= 20
    x = x.bfloat16()
    n, C, F = x.numel(), x.shape[0], x.shape[1]
    qdq("c3_channel_axis0_bf16_28672x8192", x, dict(dtype=torch.int8, mode="channel", ch_axis=0),
        3 * n + 4 * C, 3 * n + 4 * C)
    qdq("c3_channel_axis1_bf16_28672x8192", x, dict(dtype=torch.int8, mode="channel", ch_axis=1),
        3 * n + 4 * F, 3 * n + 4 * F)
    del x
    x = torch.randn(16384, 14336, device=dev, generator=g)
    x *= 0.1 + 9.9 * torch.rand(16384, 1, device=dev, generator=g)
    x = x.bfloat16()
    n = x.numel()
    qdq("c4_group128_bf16_16384x14336", x,
        dict(dtype=torch.int8, mode="group", group_size=128, ch_axis=-1),
        3 * n + 4 * (n // 128), 3 * n + 4 * (n // 128))
    del x
    if not no_w8a16:
        def w8a16_rec(M, N, K, us, us_fp16=None):
            flops = 2.0 * M * N * K
            bytes_ = N * K + 2 * N + 2 * M * K + 2 * M * N
            r = {"us": round(us, 2), "tflops": round(flops / us / 1e6, 2),
                 "mfma_frac": round(flops / (us * 1e-6) / FP16_PEAK, 4),
                 "gbs": round(bytes_ / us / 1e3, 1),
                 "hbm_frac": round(bytes_ / (us * 1e-6) / HBM_PEAK, 4)}
            if us_fp16 is not None:
                r["fp16_linear_us"] = round(us_fp16, 2)
                r["speedup_vs_fp16_linear"] = round(us_fp16 / us, 3)
            return r

        # config 5 at its three M, then the bottom of the north star's M >= 1024
        # range (1024, 1536), each next to an fp16 F.linear of the dequantized
        # weight (the runtime's GEMM library) timed the same way
        for M in (16, 256, 1024, 1536, 4096):
            xa, w = configs.c5_w8a16(M)
            N, K = w.shape
            layer = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16)
            layer.quantize(w.to(dev))
            xd = xa.to(dev)
            us = statistics.median(time_op(lambda: layer(xd), EXTRA_REPS, 2, flush))
            wd = (layer.int8_weights.half() * layer.scales[:, None]).contiguous()
            us_fp16 = statistics.median(time_op(lambda: torch.nn.functional.linear(xd, wd),
                                                EXTRA_REPS, 2, flush))
            out[f"c5_w8a16_m{M}"] = w8a16_rec(M, N, K, us, us_fp16)
            print(f"[bench] w8a16 M={M}: {us:.1f} us (fp16 F.linear {us_fp16:.1f} us)",
                  file=sys.stderr, flush=True)
            del layer, wd
            # config 5's outlier threshold (6.0) applied the LLM.int8 way: the
            # layer's opt-in activation mode routes the 6 outlier features of x
            # through the fp16 side-GEMM
            if M in (16, 256, 4096):
                lo = cuBladeW8A16LinearLayer(K, N, bias=False, dtype=torch.float16,
                                             handle_outliers=True, outlier_threshold=6.0,
                                             outlier_mode="activation")
                lo.quantize(w.to(dev), activations=xa)
                us_o = statistics.median(time_op(lambda: lo(xd), EXTRA_REPS, 2, flush))
                r = w8a16_rec(M, N, K, us_o)
                r["n_outlier_cols"] = int(lo.outlier_cols.numel())
                r["plain_us"] = round(us, 2)
                out[f"c5_w8a16_outliers_m{M}"] = r
                print(f"[bench] w8a16 outliers M={M}: {us_o:.1f} us ({r['n_outlier_cols']} "
                      f"columns through the side-GEMM)", file=sys.stderr, flush=True)
                del lo
            del xd
    return out


def load_traffic():
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        return float(d["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (the kernels "
                                   "would shard by rows, groups or output columns, one process "
                                   "per GPU)"}))
        sys.exit(2)
    import torch

    from cublade_amd import _abi
    from cublade_amd.benchmark import configs
    from cublade_amd.benchmark.core import MallFlush
    from cublade_amd.bindings.hip import quantize_per_tensor_int8
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor

    _abi.lib()
    dev = torch.device("cuda:0")
    x_cpu = configs.c2_int8_tensor()
    x = x_cpu.to(dev)
    stream = torch.cuda.current_stream(dev)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def run_steps(flush, nsteps, nwarm):
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

        # The warm-up keeps each step's outputs alive into the next step, as
        # the timed loop does, so that the caching allocator already holds
        # both generations of output blocks: an allocation that reaches
        # hipMalloc inside a timed phase waits for the device to drain and
        # shows up as idle time in that phase.
        qt = y = None
        for _ in range(max(nwarm, 2)):
            qt, y = step([], [])
        torch.cuda.synchronize()
        tq, td = [], []
        for _ in range(nsteps):
            qt, y = step(tq, td)
        torch.cuda.synchronize()
        q_ms = [a.elapsed_time(b) for a, b in tq]
        d_ms = [a.elapsed_time(b) for a, b in td]
        return qt, y, q_ms, d_ms

    clean = MallFlush(dev, mode="clean")
    w0 = time.perf_counter()
    qt, y, q_ms, d_ms = run_steps(clean, args.steps, args.warmup)
    wall = time.perf_counter() - w0
    sum_s = (sum(q_ms) + sum(d_ms)) / 1e3
    value = BYTES_STEP * args.steps / sum_s / 1e9
    quant_us = sum(q_ms) / len(q_ms) * 1e3
    deq_us = sum(d_ms) / len(d_ms) * 1e3

    dirty = MallFlush(dev, mode="dirty")
    _, _, q_ms2, d_ms2 = run_steps(dirty, args.steps, 1)
    del dirty
    quant_us2 = sum(q_ms2) / len(q_ms2) * 1e3
    deq_us2 = sum(d_ms2) / len(d_ms2) * 1e3

    # every kernel of the step, back to back on distinct buffers
    xs = [x.clone() for _ in range(ROOF_LAUNCHES)]
    quant_kernel_us = timed_rotation(torch, stream, clean, ev,
                                     [lambda t=t: quantize_per_tensor_int8(t) for t in xs])
    del xs
    qts = [dataclasses.replace(qt, data=qt.data.clone()) for _ in range(ROOF_LAUNCHES)]
    deq_kernel_us = timed_rotation(torch, stream, clean, ev,
                                   [lambda t=t: dequantize_tensor(t) for t in qts])
    del qts
    kernels = {
        "k_quant_tensor_1pass<fp16, int8>": {"bytes_per_launch": BYTES_QUANT,
                                             **_rate(BYTES_QUANT, quant_kernel_us)},
        "k_deq_tensor<int8, fp16>": {"bytes_per_launch": BYTES_DEQ,
                                     **_rate(BYTES_DEQ, deq_kernel_us)},
    }
    roof_name = max(kernels, key=lambda k: kernels[k]["us"])
    roof = kernels[roof_name]
    achieved = roof["bytes_per_launch"] / (roof["us"] * 1e-6) / 1e9
    copy = copy_ceiling(torch, dev, stream, clean, ev)
    status = _abi.tensor_quant_status(dev)

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
                   "bytes_per_step": BYTES_STEP,
                   "hbm_frac": round(value * 1e9 / HBM_PEAK, 4),
                   "cache_sweep": "clean (read-only 512 MiB sweep before each phase)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved * 1e9 / HBM_PEAK, 4),
                     "traffic": load_traffic(), "kernel": roof_name,
                     "bytes_per_launch": roof["bytes_per_launch"], "avg_launch_us": roof["us"]},
        "kernels": kernels,
        "phases": {"quant_us": round(quant_us, 2),
                   "quant_gbs": round(BYTES_QUANT / quant_us / 1e3, 2),
                   "dequant_us": round(deq_us, 2),
                   "dequant_gbs": round(BYTES_DEQ / deq_us / 1e3, 2),
                   "quant_us_median": round(statistics.median(q_ms) * 1e3, 2),
                   "dequant_us_median": round(statistics.median(d_ms) * 1e3, 2),
                   "max_step_us": round(max(a + b for a, b in zip(q_ms, d_ms)) * 1e3, 2)},
        "dirty": {"what": "the same steps after a write sweep (every cache line dirty)",
                  "value": round(BYTES_STEP / ((quant_us2 + deq_us2) * 1e-6) / 1e9, 2),
                  "quant_us": round(quant_us2, 2), "dequant_us": round(deq_us2, 2)},
        "copy_ceiling": copy,
        "exchange_status": status,
        "wall_s_incl_sweeps": round(wall, 3),
    }
    if not args.no_extras:
        ex = extras(torch, dev, args.no_w8a16)
        out["extras"] = ex
        if "c5_w8a16_m4096" in ex:
            m = ex["c5_w8a16_m4096"]
            out["w8a16_m4096_us"] = m["us"]
            out["w8a16_m4096_tflops"] = m["tflops"]
            out["w8a16_m4096_mfma_frac"] = m["mfma_frac"]
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x_cpu, qt.data, y)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
