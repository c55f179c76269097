"""Summaries of rocprofv3 results (the SQLite database rocprofv3 writes).

    # kernel durations (run: rocprofv3 --kernel-trace --stats -d DIR -o NAME -- python ...)
    python -m cublade_amd.benchmark.rocprof kernels DIR/NAME_results.db

    # HBM bytes per dispatch from counters (run once with --pmc FETCH_SIZE and once
    # with --pmc WRITE_SIZE; both counters are KiB per dispatch)
    python -m cublade_amd.benchmark.rocprof counters DIR/NAME_results.db

    # HBM bytes per launch of one kernel, calibrated against a known copy
    python -m cublade_amd.benchmark.rocprof traffic KERNEL FETCH.db WRITE.db \
        CAL_FETCH.db CAL_WRITE.db CAL_KIB

    # the same for every kernel of the runs (a text table)
    python -m cublade_amd.benchmark.rocprof traffic-all FETCH.db WRITE.db \
        CAL_FETCH.db CAL_WRITE.db CAL_KIB

    # average GPU clock per dispatch (run with --pmc GRBM_GUI_ACTIVE --kernel-trace):
    # the counter summed over its instances (one per XCD) over the dispatch's
    # duration, in MHz, divided by the instance count
    python -m cublade_amd.benchmark.rocprof clock DIR/NAME_results.db

The calibration runs profile a copy of CAL_KIB KiB (copy_calib.py); the
factor for each counter is CAL_KIB / (its mean over the copy dispatches).
Kernel names are shortened to their template signature. Output is plain
text (JSON for traffic) for profiles/.
"""
from __future__ import annotations

import re
import sqlite3
import sys
from collections import defaultdict


def _short(name: str) -> str:
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    name = re.sub(r"\(.*\)$", "", name)            # drop the parameter list
    name = name.replace("void ", "")
    return name[:110]


def kernel_stats(db: str):
    """[(kernel, calls, avg_us, min_us, max_us, total_us)] sorted by total."""
    con = sqlite3.connect(db)
    rows = con.execute("select name, duration from kernels").fetchall()
    agg = defaultdict(list)
    for name, dur in rows:
        agg[_short(name)].append(dur / 1e3)   # ns -> us
    out = [(k, len(v), sum(v) / len(v), min(v), max(v), sum(v)) for k, v in agg.items()]
    return sorted(out, key=lambda r: -r[5])


def counter_stats(db: str):
    """{(kernel, counter): [values per dispatch]} from a --pmc run."""
    con = sqlite3.connect(db)
    tabs = {r[0] for r in con.execute("select name from sqlite_master")}
    res = defaultdict(list)
    if "counters_collection" in tabs:
        q = ("select kernel_name, counter_name, sum(value) from counters_collection "
             "group by dispatch_id, counter_name")
        for k, c, v in con.execute(q):
            res[(_short(k), c)].append(v)
        return res
    # rocpd schema: pmc events joined with dispatches
    q = ("select k.name, i.name, sum(p.value) from rocpd_pmc_event p "
         "join rocpd_info_pmc i on p.pmc_id = i.id "
         "join rocpd_kernel_dispatch d on p.event_id = d.event_id "
         "join rocpd_info_kernel_symbol k on d.kernel_id = k.id "
         "group by d.id, i.name")
    for k, c, v in con.execute(q):
        res[(_short(k), c)].append(v)
    return res


def clock_stats(db: str, counter: str = "GRBM_GUI_ACTIVE", instances: int = 8):
    """{kernel: [(duration_us, MHz) per dispatch]}: the counter summed over its
    instances (GRBM_GUI_ACTIVE: one per XCD, 8 on MI355X) over the dispatch's
    duration from the kernel trace of the same run. Short dispatches read high:
    the counter's window is wider than the kernel."""
    con = sqlite3.connect(db)
    dur = dict(con.execute("select dispatch_id, duration from kernels"))
    res = defaultdict(list)
    q = ("select dispatch_id, kernel_name, sum(value) from counters_collection "
         "where counter_name = ? group by dispatch_id")
    for did, name, v in con.execute(q, (counter,)):
        d = dur.get(did)
        if d:
            res[_short(name)].append((d / 1e3, v / instances / d * 1e3))
    return res


def _mean_for(stats, kernel_sub, counter):
    vals = [v for (k, c), vs in stats.items() if kernel_sub in k and c == counter for v in vs]
    if not vals:
        raise SystemExit(f"no {counter} samples for a kernel matching {kernel_sub!r}")
    return sum(vals) / len(vals), len(vals)


def traffic(kernel, fetch_db, write_db, cal_fetch_db, cal_write_db, cal_kib):
    """Calibrated HBM bytes per launch of `kernel` (substring match)."""
    cal_kib = float(cal_kib)
    cf, _ = _mean_for(counter_stats(cal_fetch_db), "copyBuffer", "FETCH_SIZE")
    cw, _ = _mean_for(counter_stats(cal_write_db), "copyBuffer", "WRITE_SIZE")
    f, nf = _mean_for(counter_stats(fetch_db), kernel, "FETCH_SIZE")
    w, nw = _mean_for(counter_stats(write_db), kernel, "WRITE_SIZE")
    ff, fw = cal_kib / cf, cal_kib / cw
    read_b, write_b = f * ff * 1024, w * fw * 1024
    return {"kernel": kernel, "fetch_kib_raw": round(f, 1), "write_kib_raw": round(w, 1),
            "dispatches": [nf, nw], "fetch_factor": round(ff, 4), "write_factor": round(fw, 4),
            "hbm_read_bytes": int(read_b), "hbm_write_bytes": int(write_b),
            "hbm_bytes_per_launch": int(read_b + write_b)}


def traffic_all(fetch_db, write_db, cal_fetch_db, cal_write_db, cal_kib):
    """[(kernel, dispatches, read_bytes, write_bytes)] per dispatch, calibrated."""
    cal_kib = float(cal_kib)
    cf, _ = _mean_for(counter_stats(cal_fetch_db), "copyBuffer", "FETCH_SIZE")
    cw, _ = _mean_for(counter_stats(cal_write_db), "copyBuffer", "WRITE_SIZE")
    fs, ws = counter_stats(fetch_db), counter_stats(write_db)
    rows = []
    for (k, c), vals in fs.items():
        if c != "FETCH_SIZE":
            continue
        wv = ws.get((k, "WRITE_SIZE"))
        if not wv:
            continue
        rows.append((k, len(vals), sum(vals) / len(vals) * cal_kib / cf * 1024,
                     sum(wv) / len(wv) * cal_kib / cw * 1024))
    return sorted(rows, key=lambda r: -(r[2] + r[3]))


def main(argv=None):
    argv = argv if argv is not None else sys.argv[1:]
    if argv and argv[0] == "traffic" and len(argv) == 7:
        import json
        print(json.dumps(traffic(*argv[1:]), indent=1))
        return 0
    if argv and argv[0] == "traffic-all" and len(argv) == 6:
        print(f"{'kernel':110s} {'calls':>6s} {'read_MB':>10s} {'write_MB':>10s} {'total_MB':>10s}")
        for k, n, rb, wb in traffic_all(*argv[1:]):
            print(f"{k:110s} {n:6d} {rb / 1e6:10.2f} {wb / 1e6:10.2f} {(rb + wb) / 1e6:10.2f}")
        return 0
    if len(argv) == 2 and argv[0] == "clock":
        print(f"{'kernel':110s} {'calls':>6s}  duration_us / MHz per dispatch")
        for k, vals in sorted(clock_stats(argv[1]).items()):
            each = " ".join(f"{d:.1f}/{m:.0f}" for d, m in vals[:8]) + (" ..." if len(vals) > 8 else "")
            print(f"{k:110s} {len(vals):6d}  {each}")
        return 0
    if len(argv) != 2 or argv[0] not in ("kernels", "counters"):
        print(__doc__)
        return 2
    if argv[0] == "kernels":
        print(f"{'kernel':110s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s}")
        for k, n, avg, mn, mx, _ in kernel_stats(argv[1]):
            print(f"{k:110s} {n:6d} {avg:10.2f} {mn:10.2f} {mx:10.2f}")
    else:
        # Per kernel: mean, median and the values in dispatch order (the first
        # dispatch of a kernel can be an outlier: warm-up, first scratch use).
        for (k, c), vals in sorted(counter_stats(argv[1]).items()):
            avg = sum(vals) / len(vals)
            med = sorted(vals)[len(vals) // 2] if len(vals) % 2 else \
                sum(sorted(vals)[len(vals) // 2 - 1:len(vals) // 2 + 1]) / 2
            each = " ".join(f"{v:.1f}" for v in vals[:8]) + (" ..." if len(vals) > 8 else "")
            print(f"{k:110s} {c:12s} n={len(vals):4d} avg={avg:14.1f} median={med:14.1f}  [{each}]")
    return 0


if __name__ == "__main__":
    sys.exit(main())
