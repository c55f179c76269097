#!/bin/bash
# Profiles the benchmark workloads with rocprofv3 and writes text summaries.
#
#   bash cublade_amd/benchmark/profile.sh OUTDIR [RAWDIR] [PARTS]
#
# PARTS (default "bench,suite,ceil") selects the groups to run: "bench" is
# steps 1-2, "suite" steps 3-4, "ceil" step 5; each group writes its own
# summaries, so a long profile can be run as several shorter jobs.
#
# 1. kernel trace of bench.py (BASELINE configs[1] step, the roofline
#    rotations and the other configs' extras)
# 2. FETCH_SIZE and WRITE_SIZE of bench.py (one counter per run) and of a
#    256 MiB device copy (copy_calib.py) to calibrate both counters: the
#    headline kernels' HBM bytes per launch
# 3. the per-config suite: HIP-event timings from a run without the profiler
#    (suite_configs.json; the tracer's per-launch host cost would otherwise show in
#    host-bound ops), then a kernel trace, then FETCH_SIZE / WRITE_SIZE runs
#    of configs 1-5 (every suite kernel's HBM bytes per dispatch)
# 4. the GPU clock under load (GRBM_GUI_ACTIVE over each dispatch's duration)
#    and rocprof's derived MfmaUtil counter (MFMA busy cycles over active
#    cycles x SIMDs) for the MFMA kernels: W8A16 (config 5) and the dense
#    GEMM (f4)
# 5. bare stream ceilings (cublade_amd/benchmark/stream_ceiling.hip) and the
#    MFMA-only matrix-core rate (cublade_amd/benchmark/mfma_ceiling.hip)
# Summaries: OUTDIR/bench_c2_kernels.txt, OUTDIR/quant_int8_c2_traffic.json,
# OUTDIR/dequant_int8_c2_traffic.json, OUTDIR/suite_kernels.txt,
# OUTDIR/suite_traffic.txt, OUTDIR/suite_configs.json, OUTDIR/clock_grbm.txt,
# OUTDIR/mfma_util.txt,
# OUTDIR/stream_ceiling.txt, OUTDIR/mfma_ceiling.txt. Raw
# databases go to RAWDIR (default OUTDIR/raw; they total about 80 MiB), the
# programs' output to OUTDIR/logs.
# Run from the repository root on a GPU machine. Every GPU step has its own
# time limit; the script stops at the first failing step.
set -u
OUT=${1:?usage: profile.sh OUTDIR [RAWDIR] [PARTS]}
RAW=${2:-"$OUT/raw"}
PARTS=${3:-bench,suite,ceil}
want() { case ",$PARTS," in *",$1,"*) return 0 ;; *) return 1 ;; esac; }
LOGS="$OUT/logs"
mkdir -p "$RAW" "$LOGS"
export TMPDIR=/tmp
PY="python -u"
R="python -m cublade_amd.benchmark.rocprof"
BENCH_SHORT="bench.py --no-cpu --no-extras --steps 3 --warmup 1"

step() { echo "[profile] $*"; }

if want bench; then
  step "kernel trace: bench.py"
  timeout -k 10 300 rocprofv3 --kernel-trace --stats -d "$RAW/trace" -o bench -- \
    $PY bench.py --no-cpu > "$LOGS/trace.log" 2>&1 || exit $?
  step "counter FETCH_SIZE: bench.py"
  timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE --kernel-trace -d "$RAW/fetch" -o bench -- \
    $PY $BENCH_SHORT > "$LOGS/fetch.log" 2>&1 || exit $?
  step "counter WRITE_SIZE: bench.py"
  timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE --kernel-trace -d "$RAW/write" -o bench -- \
    $PY $BENCH_SHORT > "$LOGS/write.log" 2>&1 || exit $?
fi
if want bench || want suite; then
  step "counter FETCH_SIZE: 256 MiB copy"
  timeout -s KILL 60 rocprofv3 --pmc FETCH_SIZE --kernel-trace -d "$RAW/cal_fetch" -o calib -- \
    $PY -m cublade_amd.benchmark.copy_calib > "$LOGS/cal_fetch.log" 2>&1 || exit $?
  step "counter WRITE_SIZE: 256 MiB copy"
  timeout -s KILL 60 rocprofv3 --pmc WRITE_SIZE --kernel-trace -d "$RAW/cal_write" -o calib -- \
    $PY -m cublade_amd.benchmark.copy_calib > "$LOGS/cal_write.log" 2>&1 || exit $?
fi
CAL="$RAW/cal_fetch/calib_results.db $RAW/cal_write/calib_results.db 262144"
if want suite; then
  step "suite (HIP-event timing, no profiler attached)"
  timeout -k 10 500 $PY -m cublade_amd.benchmark.suite --json "$OUT/suite_configs.json" > "$LOGS/suite_plain.log" 2>&1 || exit $?
  step "kernel trace: suite"
  timeout -k 10 500 rocprofv3 --kernel-trace --stats -d "$RAW/suite" -o suite -- \
    $PY -m cublade_amd.benchmark.suite --reps 10 > "$LOGS/suite.log" 2>&1 || exit $?
  step "counter FETCH_SIZE: suite configs c1-c5"
  timeout -s KILL 300 rocprofv3 --pmc FETCH_SIZE --kernel-trace -d "$RAW/sfetch" -o suite -- \
    $PY -m cublade_amd.benchmark.suite --configs c1,c2,c3,c4,c5 --reps 3 --warmup 1 > "$LOGS/sfetch.log" 2>&1 || exit $?
  step "counter WRITE_SIZE: suite configs c1-c5"
  timeout -s KILL 300 rocprofv3 --pmc WRITE_SIZE --kernel-trace -d "$RAW/swrite" -o suite -- \
    $PY -m cublade_amd.benchmark.suite --configs c1,c2,c3,c4,c5 --reps 3 --warmup 1 > "$LOGS/swrite.log" 2>&1 || exit $?
  step "counter GRBM_GUI_ACTIVE: suite configs c2,c5,c5m,f4 (clock under load)"
  timeout -s KILL 300 rocprofv3 --pmc GRBM_GUI_ACTIVE --kernel-trace -d "$RAW/clk" -o suite -- \
    $PY -m cublade_amd.benchmark.suite --configs c2,c5,c5m,f4 --reps 3 --warmup 1 > "$LOGS/clk.log" 2>&1 || exit $?
  step "counter MfmaUtil: suite configs c5,c5m,f4"
  timeout -s KILL 300 rocprofv3 --pmc MfmaUtil --kernel-trace -d "$RAW/mfma" -o suite -- \
    $PY -m cublade_amd.benchmark.suite --configs c5,c5m,f4 --reps 3 --warmup 1 > "$LOGS/mfma.log" 2>&1 || exit $?

fi
if want ceil; then
  step "bare stream ceilings (stream_ceiling.hip)"
  /opt/rocm/bin/hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
    cublade_amd/benchmark/stream_ceiling.hip -o "$RAW/stream_ceiling" > "$LOGS/stream_ceiling_build.log" 2>&1 || exit $?
  timeout -k 10 120 "$RAW/stream_ceiling" > "$LOGS/stream_ceiling.log" 2>&1 || exit $?
  step "MFMA-only rate (mfma_ceiling.hip)"
  /opt/rocm/bin/hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
    cublade_amd/benchmark/mfma_ceiling.hip -o "$RAW/mfma_ceiling" > "$LOGS/mfma_ceiling_build.log" 2>&1 || exit $?
  timeout -k 10 120 "$RAW/mfma_ceiling" > "$LOGS/mfma_ceiling.log" 2>&1 || exit $?

fi

step "summaries"
if want bench; then
  {
    echo "# rocprofv3 kernel trace of bench.py (BASELINE configs[1] step, roofline rotations, extras)"
    echo "# command: rocprofv3 --kernel-trace --stats -d RAW/trace -o bench -- python -u bench.py --no-cpu"
    echo "# durations in microseconds"
    $R kernels "$RAW/trace/bench_results.db"
    echo
    echo "# bench.py output line under the profiler:"
    grep '"metric"' "$LOGS/trace.log"
  } > "$OUT/bench_c2_kernels.txt" || exit $?
  traffic_json() {   # KERNEL ALGO_BYTES OUTFILE
    $R traffic "$1" "$RAW/fetch/bench_results.db" "$RAW/write/bench_results.db" $CAL \
    | python -c 'import json,sys; d=json.load(sys.stdin); a=int(sys.argv[1]); d["command"]="bash cublade_amd/benchmark/profile.sh OUTDIR: rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --kernel-trace -- python -u bench.py --no-cpu --no-extras --steps 3 --warmup 1; calibration: the same counters over python -m cublade_amd.benchmark.copy_calib (256 MiB copy = 262144 KiB)"; d["algorithmic_bytes_per_launch"]=a; d["traffic_over_algorithmic"]=round(d["hbm_bytes_per_launch"]/a,4); print(json.dumps(d, indent=1))' "$2" \
    > "$3"
  }
  traffic_json "k_quant_tensor_1pass<1, false>" 201326596 "$OUT/quant_int8_c2_traffic.json" || exit $?
  traffic_json "k_deq_tensor<false, 1, 2>" 201326596 "$OUT/dequant_int8_c2_traffic.json" || exit $?
fi
if want suite; then
  {
    echo "# rocprofv3 kernel trace of the per-config suite (10 timed calls each)"
    echo "# command: rocprofv3 --kernel-trace --stats -d RAW/suite -o suite -- python -u -m cublade_amd.benchmark.suite --reps 10"
    echo "# durations in microseconds"
    $R kernels "$RAW/suite/suite_results.db"
  } > "$OUT/suite_kernels.txt" || exit $?
  {
    echo "# HBM bytes per dispatch of every kernel of suite configs c1-c5, from FETCH_SIZE and WRITE_SIZE"
    echo "# (KiB per dispatch, one counter per run) scaled by the factors a 256 MiB device copy gives"
    echo "# (its counters read back against 262144 KiB moved; see *_traffic.json for the factors)"
    echo "# commands: rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --kernel-trace -d RAW/sfetch -o suite -- python -u -m cublade_amd.benchmark.suite --configs c1,c2,c3,c4,c5 --reps 3 --warmup 1"
    $R traffic-all "$RAW/sfetch/suite_results.db" "$RAW/swrite/suite_results.db" $CAL
  } > "$OUT/suite_traffic.txt" || exit $?
  {
    echo "# average GPU clock per dispatch: GRBM_GUI_ACTIVE (one instance per XCD, summed, / 8) over the"
    echo "# dispatch's duration from the kernel trace of the same run; short dispatches read high (the"
    echo "# counter's window is wider than the kernel). W8A16 c5 (M = 16 / 256 / 768 / 1536 / 4096) and c5m"
    echo "# (M = 1024 / 2048 / 3072), N = 11008, K = 4096; c2; f4 (8192^3; Cijk_* are hipBLASLt's kernels)"
    echo "# command: rocprofv3 --pmc GRBM_GUI_ACTIVE --kernel-trace -d RAW/clk -o suite -- python -u -m cublade_amd.benchmark.suite --configs c2,c5,c5m,f4 --reps 3 --warmup 1"
    $R clock "$RAW/clk/suite_results.db" | grep -E "kernel |cbq::|Cijk"
  } > "$OUT/clock_grbm.txt" || exit $?
  {
    echo "# rocprof derived counter MfmaUtil = sum(SQ_VALU_MFMA_BUSY_CYCLES) / (max(GRBM_GUI_ACTIVE) * SIMDs) * 100,"
    echo "# per kernel: mean and median over dispatches, then the values in dispatch order (the first is the"
    echo "# suite's warm-up call): W8A16 (suite configs c5 and c5m, M = 16 / 256 / 768 / 1536 / 4096 and"
    echo "# 1024 / 2048 / 3072) and the dense GEMM (f4, 8192^3)"
    echo "# command: rocprofv3 --pmc MfmaUtil --kernel-trace -d RAW/mfma -o suite -- python -u -m cublade_amd.benchmark.suite --configs c5,c5m,f4 --reps 3 --warmup 1"
    $R counters "$RAW/mfma/suite_results.db" | grep -E "k_gemm_dma|k_stream|k_skinny|k_gemm<|k_mm_dma|Cijk"
    echo
    echo "# dispatches by W8A16 shape (N = 11008, K = 4096, config-5 operands; order: c5 then c5m):"
    echo "#   M = 16    k_stream1<1, 3>                          (weight streaming, HBM-bound)"
    echo "#   M = 256   k_gemm_dma<1, false, 2, false, 1, 2>     (172 tiles of 128 x 128, one round, no split)"
    echo "#   M = 768   k_gemm_dma<1, false, 3, false, 2, 2>     first 4 values (172 tiles of 192 rows, one wave)"
    echo "#   M = 1536  k_gemm_dma<1, true, 4, false, 2, 2>      first 4 values (256 tiles whole + 2 over 16 ranges)"
    echo "#   M = 4096  k_gemm_dma<1, false, 4, false, 2, 2>     first 4 values (688 tiles, 2.69 waves)"
    echo "#   M = 1024  k_gemm_dma<1, false, 4, false, 2, 2>     last 4 values (172 tiles of 256 rows, one wave)"
    echo "#   M = 2048  k_gemm_dma<1, false, 3, false, 2, 2>     last 4 values (473 tiles of 192 rows)"
    echo "#   M = 3072  k_gemm_dma<1, true, 4, false, 2, 2>      last 4 values (512 tiles whole + the tail split)"
    echo "# dense GEMM (f4): k_mm_dma<0, 0, ...> int8 (B [N, K] read in place, then [K, N]), k_mm_dma<1, 1, ...>"
    echo "# fp16 -> fp32; Cijk_* are hipBLASLt's kernels for torch._int_mm and torch.matmul on the same shapes"
  } > "$OUT/mfma_util.txt" || exit $?
fi
if want ceil; then
  {
    echo "# bare HBM streams with the quant / dequant access mixes (no arithmetic): the ceilings the"
    echo "# kernels' roofline fractions are read against; first the timing floor of one launch"
    echo "# command: hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops cublade_amd/benchmark/stream_ceiling.hip -o RAW/stream_ceiling && RAW/stream_ceiling"
    cat "$LOGS/stream_ceiling.log"
  } > "$OUT/stream_ceiling.txt" || exit $?
  {
    echo "# matrix-core rate with nothing but MFMAs in flight: the ceiling the GEMM kernels' TFLOP/s"
    echo "# are read against (the clock falls under MFMA load, and further with random operands)"
    echo "# command: hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops cublade_amd/benchmark/mfma_ceiling.hip -o RAW/mfma_ceiling && RAW/mfma_ceiling"
    cat "$LOGS/mfma_ceiling.log"
  } > "$OUT/mfma_ceiling.txt" || exit $?
fi
step "done"
