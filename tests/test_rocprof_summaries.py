"""The rocprofv3 summary helpers (cublade_amd/benchmark/rocprof.py) on small
synthetic databases with the tables they read (CPU)."""
from __future__ import annotations

import sqlite3

import pytest

from cublade_amd.benchmark import rocprof


def _db(path, kernels, counters):
    """kernels: [(dispatch_id, name, duration_ns)]; counters: [(dispatch_id,
    name, counter, value)] (one row per counter instance)."""
    con = sqlite3.connect(path)
    con.execute("create table kernels (dispatch_id integer, name text, duration integer)")
    con.execute("create table counters_collection (dispatch_id integer, kernel_name text, "
                "counter_name text, value real)")
    con.executemany("insert into kernels values (?, ?, ?)", kernels)
    con.executemany("insert into counters_collection values (?, ?, ?, ?)", counters)
    con.commit()
    con.close()
    return str(path)


K1 = "void cbq::(anonymous namespace)::k_gemm_dma<1, false, 4, false, 2, 2>(cbq::GemmArgs)"
K2 = "__amd_rocclr_copyBuffer"


def test_kernel_stats(tmp_path):
    db = _db(tmp_path / "k.db", [(1, K1, 300_000), (2, K1, 320_000), (3, K2, 10_000)], [])
    rows = rocprof.kernel_stats(db)
    assert rows[0][0] == "cbq::k_gemm_dma<1, false, 4, false, 2, 2>"
    assert rows[0][1:5] == (2, 310.0, 300.0, 320.0)
    assert rows[1][0] == K2 and rows[1][1] == 1


def test_counter_and_clock_stats(tmp_path):
    # GRBM_GUI_ACTIVE has one instance per XCD: 8 rows per dispatch
    cnt = [(1, K1, "GRBM_GUI_ACTIVE", 480_000.0) for _ in range(8)]
    cnt += [(2, K1, "GRBM_GUI_ACTIVE", 512_000.0) for _ in range(8)]
    db = _db(tmp_path / "c.db", [(1, K1, 300_000), (2, K1, 320_000)], cnt)
    stats = rocprof.counter_stats(db)
    assert stats[("cbq::k_gemm_dma<1, false, 4, false, 2, 2>", "GRBM_GUI_ACTIVE")] == \
        [8 * 480_000.0, 8 * 512_000.0]
    clk = rocprof.clock_stats(db)["cbq::k_gemm_dma<1, false, 4, false, 2, 2>"]
    # 480000 cycles in 300 us: 1600 MHz; 512000 in 320 us: 1600 MHz
    assert clk == [pytest.approx((300.0, 1600.0)), pytest.approx((320.0, 1600.0))]


def test_traffic_calibration(tmp_path):
    # the copy moves 1024 KiB and its counters read 512 (fetch) and 2048 (write):
    # factors 2 and 0.5
    cal_f = _db(tmp_path / "cf.db", [(1, K2, 1000)], [(1, K2, "FETCH_SIZE", 512.0)])
    cal_w = _db(tmp_path / "cw.db", [(1, K2, 1000)], [(1, K2, "WRITE_SIZE", 2048.0)])
    f = _db(tmp_path / "f.db", [(1, K1, 1000)], [(1, K1, "FETCH_SIZE", 100.0)])
    w = _db(tmp_path / "w.db", [(1, K1, 1000)], [(1, K1, "WRITE_SIZE", 40.0)])
    t = rocprof.traffic("k_gemm_dma", f, w, cal_f, cal_w, 1024)
    assert t["fetch_factor"] == 2.0 and t["write_factor"] == 0.5
    assert t["hbm_read_bytes"] == 200 * 1024 and t["hbm_write_bytes"] == 20 * 1024
    assert t["hbm_bytes_per_launch"] == 220 * 1024
